// GEMM family for gfx950: mm / addmm / bmm.
//
// Large bf16 / f16 GEMMs (K % 128 == 0, >= 128 output tiles of 256x256):
// `gemm_dma_kernel` -- 256x256x64 work-group tiles, 8 waves (2 per SIMD) of
// 128x64, 32x32x16 MFMAs, two LDS stages filled by buffer_load ... lds
// (direct global -> LDS DMA, no VGPR staging).  Row-major B stays
// N-contiguous in LDS and is read with ds_read_b64_tr_b16; A and a
// K-contiguous B are read with ds_read_b128.  Each LDS stage is its own
// __shared__ array so the compiler need not make LDS reads wait for DMA that
// targets the other stage.
//
// Everything else bf16 / f16 (any M, N; K % 8 == 0): `gemm_mfma_kernel` --
// BM x BN x 64 tiles (256x256 or 128x128), 4 waves, register-staged global
// loads (a row-major B is transposed in registers on its way into LDS), two
// LDS stages, optional split-K whose fp32 partials `splitk_reduce_kernel`
// sums in split order (deterministic).
//
// Work-group ids are remapped so that neighbouring output tiles run on the
// same XCD (dispatch is round-robin over the 8 XCDs, each with its own L2)
// and are visited in groups of 8 tile-rows.
//
// f32 / f64 and unaligned operands take `gemm_simt_kernel`, a plain
// LDS-tiled kernel with the same epilogue.
//
// Semantics follow aten mm / addmm / bmm (the reference's fallthrough and
// test oracle, kuipy/kuiops.py:403-564, tests/test_jit_ops.py:51-112).
#include <stdlib.h>

#include <type_traits>

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
    int vec_store;         // gemm_dma_kernel: 16-byte row-segment epilogue (ldo, N % 8 == 0, aligned out)
    int raster;            // tile order within a batch entry: 0 = groups of 8 tile-rows, 1 = row by row
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

// Batched form: the linear id runs over batch x tiles; after the XCD remap
// each batch entry's tiles are contiguous (so one XCD's L2 holds its A and
// B), and tiles are grouped by 8 tile-rows within the entry.
__device__ __forceinline__ void tile_coords_batched(int bid, int nblocks, int tiles_m, int tiles_n,
                                                    int &tm, int &tn, int &bz, int raster = 0) {
    const int xcd = bid & 7, idx = bid >> 3;
    const int q = nblocks >> 3, r = nblocks & 7;
    const int pid = xcd * q + (xcd < r ? xcd : r) + idx;
    const int per = tiles_m * tiles_n;
    bz = pid / per;
    const int t = pid - bz * per;
    if (raster) {
        // row by row: the tiles one XCD runs at once lie side by side, so
        // their 512-byte row segments of the output form whole rows
        tm = t / tiles_n;
        tn = t - tm * tiles_n;
        return;
    }
    const int G = 8;
    const int width = G * tiles_n;
    const int group = t / width;
    const int first_m = group * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in_group = t - group * width;
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

// ------------------------------------------------------------------------
// gfx950 LDS-DMA kernel: 256x256x64 tiles, 4 waves (2x2), each wave 128x128
// built from 32x32x16 MFMAs.  Global tiles go straight into LDS with
// global_load_lds_dwordx4 (no VGPR staging, no ds_write): the LDS position a
// lane fills is fixed (base + 16 * lane), so the XOR swizzle is applied by
// choosing which 16-byte chunk each lane fetches.
//   * A ([M, K], K contiguous) and a K-contiguous B: LDS rows of 64 k (128 B),
//     chunk c stored at position c ^ (row & 7); operands are ds_read_b128.
//   * Row-major B ([K, N]): kept N-contiguous in LDS (rows of 256 n, 512 B),
//     chunk c of row k stored at c ^ fB(k); the MFMA operand (8 consecutive k
//     of one column) is assembled by two ds_read_b64_tr_b16: within each group
//     of 16 lanes, source lane q addresses row k0 + q/4, columns 4*(q%4)..+3,
//     and output lane p receives rows k0..k0+3 of column p.
// Requires K % 128 == 0 (the K loop is unrolled by the two LDS stages);
// rows / columns past M / N are clamped on load and dropped on store.
__device__ __forceinline__ int swzB(int k) { return ((k & 3) | (((k >> 3) & 1) << 2)) << 2; }

typedef __attribute__((address_space(3))) char lds_char;
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Generic -> LDS address-space cast.  A direct cast keeps the pointer's
// provenance (an integer round trip would hide which LDS array it points
// into, and the compiler would then make every LDS read wait for all
// in-flight LDS-DMA loads).
__device__ __forceinline__ lds_char *to_lds(const void *p) {
    return (lds_char *)(const_cast<void *>(p));
}

// One global_load_lds_dwordx4: 16 bytes from `src` per lane into
// dst + 16 * lane (dst is wave-uniform).  The source must reach the builtin
// as `const void *`: a typed pointer makes the host compilation pass drop
// the kernel's launch stub without a diagnostic.
__device__ __forceinline__ void dma16(const void *src, const void *dst) {
    __builtin_amdgcn_global_load_lds(src, to_lds(dst), 16, 0, 0);
}

// Buffer-resource form of the same copy: a wave-uniform descriptor (SGPRs),
// a per-lane 32-bit byte offset and a uniform byte offset, so the K-step
// advance costs no per-lane address registers.  Reads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const void *dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)to_lds(dst), 16,
                                             (int)voff, (int)soff, 0, 0);
}

// Epilogue of one 32x32 accumulator tile: lane holds column `col` and rows
// row0 + 8 * (e / 4) + 4 * lk + e % 4.  The addend kind is wave-uniform.
template <typename Tout>
__device__ __forceinline__ void store_tile32(const GemmArgs &a, const f32x16 &acc, int64_t row0, int64_t col,
                                             int lk) {
    if (col >= a.N) return;
    Tout *out = reinterpret_cast<Tout *>(a.out) + row0 * a.ldo + col;
    const Tout *cin = reinterpret_cast<const Tout *>(a.cin);
    const bool full_rows = row0 + 32 <= a.M;
    float add[16];
    if (a.c_kind == KUIOPS_C_ROW) {
        const float b = a.beta * to_f32(cin[col]);
#pragma unroll
        for (int e = 0; e < 16; ++e) add[e] = b;
    } else if (a.c_kind == KUIOPS_C_FULL) {
        const Tout *c = cin + row0 * a.ldcin + col;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = (e >> 2) * 8 + lk * 4 + (e & 3);
            add[e] = (full_rows || row0 + r < a.M) ? a.beta * to_f32(c[(int64_t)r * a.ldcin]) : 0.f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) add[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int r = (e >> 2) * 8 + lk * 4 + (e & 3);
        if (full_rows || row0 + r < a.M) out[(int64_t)r * a.ldo] = from_f32<Tout>(a.alpha * acc[e] + add[e]);
    }
}

// vmcnt-only wait (expcnt / lgkmcnt left at their maxima), N < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <typename T, bool BCOL, typename Tout, int WM, int WN, int BK, int NS>
__global__ __launch_bounds__(WM * WN * 64) void gemm_dma_kernel(GemmArgs a) {
    constexpr int BM = 256, BN = 256;
    constexpr int NW = WM * WN;                    // waves
    constexpr int WTM = BM / WM, WTN = BN / WN;    // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;    // 32x32 tiles per wave
    constexpr int KK = BK / 16;                    // MFMA k-steps per stage
    constexpr int RB = BK * 2;                     // bytes per K-contiguous LDS row
    constexpr int RPB = 1024 / RB;                 // such rows per 1 KB DMA block
    constexpr int CPR = BK / 8;                    // 16-byte chunks per such row
    constexpr int SBYTES = BM * BK * 2;            // bytes per operand per stage (BM == BN)
    constexpr int DPW = SBYTES / 1024 / NW;        // DMA blocks per wave, per operand, per stage
    static_assert(BK == 32 || BK == 64, "BK");
    static_assert(NS >= 2 && NS <= 4, "stages");
    static_assert(DPW >= 1, "DMA split");
    typedef typename Mfma<T>::frag frag;
    // One array per operand and stage: the compiler tracks LDS-DMA writes per
    // underlying object, so reads of one stage need not wait for the DMA that
    // is filling another.
    __shared__ __attribute__((aligned(1024))) char sA0[SBYTES], sB0[SBYTES];
    __shared__ __attribute__((aligned(1024))) char sA1[SBYTES], sB1[SBYTES];
    __shared__ __attribute__((aligned(1024))) char sA2[NS > 2 ? SBYTES : 16], sB2[NS > 2 ? SBYTES : 16];
    __shared__ __attribute__((aligned(1024))) char sA3[NS > 3 ? SBYTES : 16], sB3[NS > 3 ? SBYTES : 16];
    char *const SA[4] = {sA0, sA1, sA2, sA3};
    char *const SB[4] = {sB0, sB1, sB2, sB3};

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn, bz;
    tile_coords_batched(blockIdx.x, gridDim.x, a.tiles_m, a.tiles_n, tm, tn, bz, a.raster);
    a.A = reinterpret_cast<const T *>(a.A) + bz * a.stride_a;
    a.B = reinterpret_cast<const T *>(a.B) + bz * a.stride_b;
    a.out = reinterpret_cast<Tout *>(a.out) + bz * a.stride_o;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int nk = (int)(a.K / BK);                // multiple of NS

    // K-contiguous rows: chunk c of row r sits at position c ^ swzK(r).
    // 64 LDS banks: a ds_read_b128 serves 16 lanes (16 consecutive rows) per
    // cycle, so the 16 (row parity, position) pairs of those rows must differ.
    auto swzK = [](int r) { return CPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); };

    // Uniform tile bases plus 32-bit per-lane byte offsets (clamped rows /
    // columns past M / N read valid memory; their results are not stored).
    const char *baseA = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.A) + m0 * a.lda);
    const char *baseB = BCOL ? reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.B) + n0 * a.ldb)
                             : reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.B) + n0);
    uint32_t goffA[DPW], goffB[DPW];
#pragma unroll
    for (int j = 0; j < DPW; ++j) {
        const int blk = wave * DPW + j;
        const int r = blk * RPB + lane / CPR;
        const int c = (lane % CPR) ^ swzK(r);
        goffA[j] = (uint32_t)((min((int64_t)r, a.M - 1 - m0) * a.lda + c * 8) * 2);
        if constexpr (BCOL) {
            goffB[j] = (uint32_t)((min((int64_t)r, a.N - 1 - n0) * a.ldb + c * 8) * 2);
        } else {
            const int kr = blk * 2 + (lane >> 5);   // B rows are 512 B: 2 per block
            const int cb = (lane & 31) ^ swzB(kr);
            goffB[j] = (uint32_t)(((int64_t)kr * a.ldb + min((int64_t)cb * 8, a.N - 8 - n0)) * 2);
        }
    }
    const int64_t stepA = (int64_t)BK * 2;                          // bytes per K step
    const int64_t stepB = BCOL ? (int64_t)BK * 2 : (int64_t)BK * a.ldb * 2;

    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(baseA, 0xffffffffu);
    const __amdgpu_buffer_rsrc_t rsB = make_rsrc(baseB, 0xffffffffu);
    auto issue = [&](int kt, char *sa, char *sb) __attribute__((always_inline)) {
        const uint32_t ka = (uint32_t)(kt * stepA), kb = (uint32_t)(kt * stepB);
#pragma unroll
        for (int j = 0; j < DPW; ++j) dma16_buf(rsA, goffA[j], ka, sa + (wave * DPW + j) * 1024);
#pragma unroll
        for (int j = 0; j < DPW; ++j) dma16_buf(rsB, goffB[j], kb, sb + (wave * DPW + j) * 1024);
    };

    // LDS byte offsets of this lane's operand fragments.
    const int lrow = lane & 31, lk = lane >> 5;
    const int G = lane >> 4, q = lane & 15;
    int offA[KK];                // per kk; tile i adds i * 32 rows
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int r = wm * WTM + lrow;
        offA[kk] = r * RB + (((2 * kk + lk) ^ swzK(r)) << 4);
    }
    int offB[BCOL ? KK : TN];    // K-contiguous B: per kk like A; row-major B: per tile j
    if constexpr (BCOL) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const int r = wn * WTN + lrow;
            offB[kk] = r * RB + (((2 * kk + lk) ^ swzK(r)) << 4);
        }
    } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int kr = 8 * (G >> 1) + (q >> 2);                 // + 16 kk + 4 h
            const int n = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (q & 3);
            offB[j] = kr * 512 + (((n >> 3) ^ swzB(kr)) << 4) + ((n >> 2) & 1) * 8;
        }
    }

    auto load_frags = [&](const char *sa, const char *sb, int kk, frag *fa, frag *fb) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
            fa[i] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sa + offA[kk] + i * 32 * RB));
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if constexpr (BCOL) {
                fb[j] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sb + offB[kk] + j * 32 * RB));
            } else {
                const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512));
                const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512 + 4 * 512));
                const u32x2 h0 = __builtin_bit_cast(u32x2, t0), h1 = __builtin_bit_cast(u32x2, t1);
                fb[j] = as_frag<frag>(u32x4{h0[0], h0[1], h1[0], h1[1]});
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

    // MFMAs of one stage; fragments double-buffered (reads of kk + 1 are
    // issued before the MFMAs of kk).
    auto compute = [&](const char *sa, const char *sb) {
        frag fa[2][TM], fb[2][TN];
        load_frags(sa, sb, 0, fa[0], fb[0]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (kk + 1 < KK) load_frags(sa, sb, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = Mfma<T>::m32(fa[kk & 1][i], fb[kk & 1][j], acc[i][j]);
        }
    };

    // Pipeline: stages 0..NS-2 are in flight before the loop.  Step kt waits
    // for its own stage (the DMA of the younger stages may stay in flight),
    // synchronises the work-group, refills the stage consumed at step kt - 1
    // with step kt + NS - 1, then computes.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        if (s < nk) issue(s, SA[s], SB[s]);
    for (int kt0 = 0; kt0 < nk; kt0 += NS) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int kt = kt0 + s;
            const int younger = min(NS - 2, nk - 1 - kt);      // stages issued after kt
            if (younger >= 2) wait_vmcnt<2 * 2 * DPW>();
            else if (younger == 1) wait_vmcnt<2 * DPW>();
            else wait_vmcnt<0>();
            __syncthreads();
            if (kt + NS - 1 < nk) issue(kt + NS - 1, SA[(s + NS - 1) % NS], SB[(s + NS - 1) % NS]);
            compute(SA[s], SB[s]);
        }
    }

    if constexpr (sizeof(Tout) == 2 && WM == 2 && WN == 4 && TM * 32 == WTM && 32 * (BN * 2 + 16) <= SBYTES) {
        if (a.vec_store) {
            // Staged epilogue: the tile goes out as whole 512-byte row segments
            // (16 bytes per lane) instead of the accumulator layout's 64-byte
            // pieces.  Pass p stages rows 32p.. of each wave row (wm) band in
            // the freed stage buffers (sA0 for wm = 0, sB0 for wm = 1), rows
            // 528 bytes apart (16 bytes of padding: the two row halves a
            // store instruction covers fall on different banks).
            constexpr int RS = BN * 2 + 16;
            static_assert(32 * RS <= SBYTES, "staging band");
            char *band = wm == 0 ? sA0 : sB0;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                __syncthreads();                 // stage buffers (or the previous band) free
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int64_t col = n0 + wn * WTN + j * 32 + lrow;
                    const int64_t row0 = m0 + wm * WTM + i * 32;
                    float add[16];
                    if (a.c_kind == KUIOPS_C_ROW) {
                        const float bv = col < a.N ? a.beta * to_f32(reinterpret_cast<const Tout *>(a.cin)[col]) : 0.f;
#pragma unroll
                        for (int e = 0; e < 16; ++e) add[e] = bv;
                    } else if (a.c_kind == KUIOPS_C_FULL) {
                        const Tout *c = reinterpret_cast<const Tout *>(a.cin);
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const int64_t r = row0 + (e >> 2) * 8 + lk * 4 + (e & 3);
                            add[e] = (r < a.M && col < a.N) ? a.beta * to_f32(c[r * a.ldcin + col]) : 0.f;
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 16; ++e) add[e] = 0.f;
                    }
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int r = (e >> 2) * 8 + lk * 4 + (e & 3);
                        *reinterpret_cast<Tout *>(band + r * RS + (wn * WTN + j * 32 + lrow) * 2) =
                            from_f32<Tout>(a.alpha * acc[i][j][e] + add[e]);
                    }
                }
                __syncthreads();
                // 2 bands x 32 rows x 32 chunks of 16 bytes over 512 threads
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int idx = rr * NW * 64 + tid;
                    const int bnd = idx >> 10, row = (idx >> 5) & 31, ch = idx & 31;
                    const int64_t grow = m0 + bnd * WTM + i * 32 + row;
                    const int64_t gcol = n0 + ch * 8;
                    const u32x4 v = *reinterpret_cast<const u32x4 *>((bnd ? sB0 : sA0) + row * RS + ch * 16);
                    if (grow < a.M && gcol < a.N)
                        // streaming store: the output is not read again here
                        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(reinterpret_cast<Tout *>(a.out) + grow * a.ldo + gcol));
                }
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            store_tile32<Tout>(a, acc[i][j], m0 + wm * WTM + i * 32, n0 + wn * WTN + j * 32 + lrow, lk);
}

// Uniform (wave-invariant) pointer kept in SGPRs: buffer descriptors built
// from it need no per-lane waterfall loop around each DMA.
__device__ __forceinline__ const char *uniform_ptr(const char *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const char *>(((uint64_t)hi << 32) | lo);
}

// ------------------------------------------------------------------------
// gemm_stream_kernel: short-K batched GEMMs (K <= 128, so a tile's whole K
// fits the two 64-k LDS stages; bmm 32 x 2048x128x2048 writes 268 MB and
// reads 33 MB, so the output stores bound it).  A persistent grid of one
// 8-wave work-group per CU walks the tiles in row-by-row order (at step i
// the grid holds tiles 256 i .. 256 i + 255, whose 512-byte row segments
// make whole output rows).  The DMA of the next tile is issued before the
// current tile's output stores, so each CU loads and stores at the same
// time; the waits leave the stores in flight (vmcnt counts the 16 stores of
// a tile, younger than the DMA) and the barriers are bare s_barrier (a
// __syncthreads() fence would wait for the stores).  Operand layouts and
// fragments are gemm_dma_kernel's (2 x 4 waves of 128x64); the output goes
// through a separate 32 KB LDS band (two 32-row bands of 512-byte rows,
// 16-byte chunks XOR-swizzled by row), so the stage buffers are free for
// the next tile's DMA.  Full 256x256 tiles, 16-bit output, no addend; B
// row-major (transposing fragment reads) or column-major (B^T rows staged
// and read like A's).
template <typename T, bool BCOL, typename Tout, int NK>
__global__ __launch_bounds__(512) void gemm_stream_kernel(GemmArgs a, int total_tiles) {
    constexpr int BK = 64, WTM = 128, WTN = 64, TM = 4, TN = 2, KK = BK / 16;
    constexpr int RB = BK * 2, RPB = 1024 / RB, CPR = BK / 8;
    constexpr int SBYTES = 256 * BK * 2;           // 32 KB per operand per stage
    constexpr int DPW = SBYTES / 1024 / 8;         // 1 KB DMA blocks per wave per operand
    constexpr int NSTORE = TM * 4;                 // 16-byte output stores per thread per tile
    typedef typename Mfma<T>::frag frag;
    __shared__ __attribute__((aligned(1024))) char sA0[SBYTES], sB0[SBYTES], sA1[SBYTES], sB1[SBYTES];
    __shared__ __attribute__((aligned(1024))) char sOut[2 * 32 * 512];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / 4, wn = wave % 4;
    const int per = a.tiles_m * a.tiles_n;
    // work-group -> first tile: ids on one XCD (dispatched round-robin) take a
    // contiguous range of each step's 256 tiles
    const int G = gridDim.x, bid = blockIdx.x;
    const int pid = __builtin_amdgcn_readfirstlane((bid & 7) * (G >> 3) + min(bid & 7, G & 7) + (bid >> 3));
    auto swzK = [](int r) { return (r >> 1) & 7; };

    uint32_t goffA[DPW], goffB[DPW];
#pragma unroll
    for (int j = 0; j < DPW; ++j) {
        const int blk = wave * DPW + j;
        const int r = blk * RPB + lane / CPR;
        const int c = (lane % CPR) ^ swzK(r);
        goffA[j] = (uint32_t)((r * a.lda + c * 8) * 2);
        if constexpr (BCOL) {
            goffB[j] = (uint32_t)((r * a.ldb + c * 8) * 2);     // B^T rows: A's layout
        } else {
            const int kr = blk * 2 + (lane >> 5);
            const int cb = (lane & 31) ^ swzB(kr);
            goffB[j] = (uint32_t)((kr * a.ldb + cb * 8) * 2);
        }
    }
    const uint32_t stepB = BCOL ? (uint32_t)(BK * 2) : (uint32_t)(BK * a.ldb * 2);
    // both K stages of tile t (the tile's operand bases are uniform)
    // stage st (0 or 1) of tile t
    auto issue = [&](int t, int st) __attribute__((always_inline)) {
        const int bz = t / per, rr = t - bz * per;
        const int tm = rr / a.tiles_n, tn = rr - tm * a.tiles_n;
        const char *ba = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.A) + bz * a.stride_a +
                                                        (int64_t)tm * 256 * a.lda);
        const char *bb = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.B) + bz * a.stride_b +
                                                        (int64_t)tn * 256 * (BCOL ? a.ldb : 1));
        const __amdgpu_buffer_rsrc_t rsA = make_rsrc(uniform_ptr(ba), 0xffffffffu);
        const __amdgpu_buffer_rsrc_t rsB = make_rsrc(uniform_ptr(bb), 0xffffffffu);
        if (st == 0) {
#pragma unroll
            for (int j = 0; j < DPW; ++j) {
                dma16_buf(rsA, goffA[j], 0, sA0 + (wave * DPW + j) * 1024);
                dma16_buf(rsB, goffB[j], 0, sB0 + (wave * DPW + j) * 1024);
            }
        } else {
#pragma unroll
            for (int j = 0; j < DPW; ++j) {
                dma16_buf(rsA, goffA[j], BK * 2, sA1 + (wave * DPW + j) * 1024);
                dma16_buf(rsB, goffB[j], stepB, sB1 + (wave * DPW + j) * 1024);
            }
        }
    };

    const int lrow = lane & 31, lk = lane >> 5;
    const int Gq = lane >> 4, q = lane & 15;
    int offA[KK], offB[TN];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int r = wm * WTM + lrow;
        offA[kk] = r * RB + (((2 * kk + lk) ^ swzK(r)) << 4);
    }
    int offKc[KK];                                  // (column-major B) chunk of k-step kk
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) offKc[kk] = ((2 * kk + lk) ^ swzK(lrow)) << 4;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        if constexpr (BCOL) {
            // B^T row wn * WTN + 32 j + lrow in A's layout; its k-chunk
            // offset is offKc (the swizzle repeats every 16 rows)
            offB[j] = (wn * WTN + j * 32 + lrow) * RB;
        } else {
            const int kr = 8 * (Gq >> 1) + (q >> 2);
            const int n = wn * WTN + j * 32 + 16 * (Gq & 1) + 4 * (q & 3);
            offB[j] = kr * 512 + (((n >> 3) ^ swzB(kr)) << 4) + ((n >> 2) & 1) * 8;
        }
    }
    auto load_frags = [&](const char *sa, const char *sb, int kk, frag *fa, frag *fb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
            fa[i] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sa + offA[kk] + i * 32 * RB));
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if constexpr (BCOL) {
                fb[j] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sb + offB[j] + offKc[kk]));
                continue;
            }
            const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512));
            const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512 + 4 * 512));
            const u32x2 h0 = __builtin_bit_cast(u32x2, t0), h1 = __builtin_bit_cast(u32x2, t1);
            fb[j] = as_frag<frag>(u32x4{h0[0], h0[1], h1[0], h1[1]});
        }
    };
    f32x16 acc[TM][TN];
    auto compute = [&](const char *sa, const char *sb) __attribute__((always_inline)) {
        frag fa[2][TM], fb[2][TN];
        load_frags(sa, sb, 0, fa[0], fb[0]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (kk + 1 < KK) load_frags(sa, sb, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::m32(fb[kk & 1][j], fa[kk & 1][i], acc[i][j]);
        }
    };

    // One tile: its DMA has landed (the caller waited), MFMAs, then the DMA
    // of tile `next` (the last tile again when there is none: the stage
    // buffers are not read after the loop, and no DMA is conditional, so the
    // compiler's waits stay those below), then this tile's output.
    auto tile = [&](int t, int next) __attribute__((always_inline)) {
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
        // each stage is refilled with the next tile's as soon as every wave
        // has read it (stage 0 under stage 1's MFMAs)
        compute(sA0, sB0);
        __builtin_amdgcn_s_waitcnt(0xc07f);        // this wave's LDS reads are done
        __builtin_amdgcn_s_barrier();              // (every wave's): stage 0 is free
        issue(next, 0);
        if constexpr (NK > 1) {
            compute(sA1, sB1);
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_s_barrier();
            issue(next, 1);
        }
        // epilogue: per accumulator row band i, the two 32-row bands (wm =
        // 0, 1) through sOut, then 512-byte row segments to memory
        const int bz = t / per, rr = t - bz * per;
        const int tm = rr / a.tiles_n, tn = rr - tm * a.tiles_n;
        Tout *out = reinterpret_cast<Tout *>(a.out) + bz * a.stride_o;
        const int64_t m0 = (int64_t)tm * 256, n0 = (int64_t)tn * 256;
        char *band = sOut + wm * 32 * 512;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            __builtin_amdgcn_s_waitcnt(0xc07f);    // this wave's reads of the previous band are done
            __builtin_amdgcn_s_barrier();
            // (operands swapped in the MFMA: a lane holds row lrow of the band
            // and 4 consecutive columns per 8-column group, one 8-byte write)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c0 = wn * WTN + j * 32 + 8 * g + 4 * lk;   // first of the 4 columns
                    typedef Tout t4 __attribute__((ext_vector_type(4)));
                    t4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = from_f32<Tout>(a.alpha * acc[i][j][4 * g + e]);
                    *reinterpret_cast<u32x2 *>(band + lrow * 512 + (((c0 >> 3) ^ lrow) << 4) + lk * 8) =
                        __builtin_bit_cast(u32x2, w);
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);    // this wave's band writes are done
            __builtin_amdgcn_s_barrier();
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int idx = u * 512 + tid;                       // 2 bands x 32 rows x 32 chunks
                const int bnd = idx >> 10, r = (idx >> 5) & 31, ch = idx & 31;
                const u32x4 v = *reinterpret_cast<const u32x4 *>(sOut + bnd * 32 * 512 + r * 512 + ((ch ^ r) << 4));
                __builtin_nontemporal_store(
                    v, reinterpret_cast<u32x4 *>(out + (m0 + bnd * WTM + i * 32 + r) * a.ldo + n0 + ch * 8));
            }
        }
    };
    // (the host launches at most total_tiles work-groups: pid < total_tiles)
    const int last = total_tiles - 1;
    issue(pid, 0);
    if constexpr (NK > 1) issue(pid, 1);
    wait_vmcnt<0>();
    for (int t = pid; t < total_tiles; t += G) {
        wait_vmcnt<NSTORE>();          // this tile's DMA; the previous tile's stores stay in flight
        tile(t, min(t + G, last));
    }

}

// ------------------------------------------------------------------------
// gemm_wave_kernel: 256x256x64 work-group tiles, 4 waves (one per SIMD),
// each wave a 128x128 quarter built from 32x32x16 MFMAs whose 256 fp32
// accumulators live in AGPRs.  Against the 8-wave gemm_dma_kernel (128x64
// per wave) each LDS fragment feeds two MFMAs instead of 1.5, which cuts the
// LDS reads per stage from 192 KB to 128 KB: LDS bandwidth (reads plus the
// DMA's writes) is what bounds this loop.  With one wave per SIMD nothing
// hides latency, so the schedule is explicit:
//   * the MFMAs of k-step kk run with the fragments of kk + 1 being read
//     under them (one LDS read issued after each MFMA);
//   * before the last k-step of a stage each wave waits for its own DMA of
//     the next stage, the work-group meets at one bare s_barrier (every wave
//     has then read the current stage), and the next stage's first
//     fragments plus half of the DMA refill of the current stage's buffers
//     with stage s + 2 are issued under the last k-step's MFMAs, the other
//     half under the next stage's first k-step (8 DMA instructions per
//     k-step at most: 99 against 108 us at 4096^3 for all 16 in one);
//   * the loop is unrolled over the two LDS stages with the last two stages
//     peeled, so no conditional DMA sits inside it (the compiler's wait
//     insertion is not path-sensitive: a conditional refill makes it wait
//     for every DMA before each stage's first LDS read).
// The MFMA operands are swapped (the B fragment is the first operand), so a
// lane's accumulator holds one output row and 4 consecutive columns per
// 8-column group: the epilogue writes 8-byte runs into an LDS image of the
// tile (16-byte chunks XOR-swizzled by row) and the work-group stores whole
// 512-byte row segments.  Loads and the LDS layouts are gemm_dma_kernel's.

template <typename T, bool BCOL, typename Tout, bool FULLC>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_wave_kernel(GemmArgs a) {
    constexpr int BK = 64, SB = 256 * BK * 2;      // bytes per operand per stage
    typedef typename Mfma<T>::frag frag;
    __shared__ __attribute__((aligned(1024))) char sA0[SB], sB0[SB], sA1[SB], sB1[SB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn, bz;
    tile_coords_batched(blockIdx.x, gridDim.x, a.tiles_m, a.tiles_n, tm, tn, bz);
    // (uniform: kept in SGPRs, so the epilogue's addressing does not hold
    // VGPRs across the K loop, which would spill)
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    bz = __builtin_amdgcn_readfirstlane(bz);
    const T *Ab = reinterpret_cast<const T *>(a.A) + bz * a.stride_a;
    const T *Bb = reinterpret_cast<const T *>(a.B) + bz * a.stride_b;
    const int64_t M = a.M, N = a.N, lda = a.lda, ldb = a.ldb, ldo = a.ldo, ldcin = a.ldcin;
    const int c_kind = a.c_kind, vec_store = a.vec_store;
    const float alpha = a.alpha, beta = a.beta;
    const int64_t m0 = (int64_t)tm * 256, n0 = (int64_t)tn * 256;
    const int nk = (int)(a.K / BK);                // even, >= 8 (K % 128 == 0, K >= 512)
    auto swzK = [](int r) { return (r >> 1) & 7; };

    // DMA: per stage and operand 32 blocks of 1 KB, 8 per wave.  Rows /
    // columns past M / N are clamped (valid memory, results not stored).
    const char *baseA = reinterpret_cast<const char *>(Ab + m0 * lda);
    const char *baseB = BCOL ? reinterpret_cast<const char *>(Bb + n0 * ldb) : reinterpret_cast<const char *>(Bb + n0);
    uint32_t goffA[8], goffB[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int blk = wave * 8 + j;
        const int r = blk * 8 + (lane >> 3);
        const int c = (lane & 7) ^ swzK(r);
        goffA[j] = (uint32_t)((min((int64_t)r, M - 1 - m0) * lda + c * 8) * 2);
        if constexpr (BCOL) {
            goffB[j] = (uint32_t)((min((int64_t)r, N - 1 - n0) * ldb + c * 8) * 2);
        } else {
            const int kr = blk * 2 + (lane >> 5);
            const int cb = (lane & 31) ^ swzB(kr);
            goffB[j] = (uint32_t)(((int64_t)kr * ldb + min((int64_t)cb * 8, N - 8 - n0)) * 2);
        }
    }
    const uint32_t stepA = BK * 2;
    const uint32_t stepB = BCOL ? (uint32_t)(BK * 2) : (uint32_t)(BK * ldb * 2);
    // (the bases are uniform; readfirstlane keeps the descriptors in SGPRs,
    // where the DMA needs them, instead of a per-lane waterfall loop)
    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(uniform_ptr(baseA), 0xffffffffu);
    const __amdgpu_buffer_rsrc_t rsB = make_rsrc(uniform_ptr(baseB), 0xffffffffu);
    // DMA blocks j0 .. j1 - 1 of both operands of stage kt
    auto issue = [&](int kt, char *sa, char *sb, int j0, int j1) __attribute__((always_inline)) {
        const uint32_t ka = (uint32_t)kt * stepA, kb = (uint32_t)kt * stepB;
#pragma unroll
        for (int j = j0; j < j1; ++j) {
            dma16_buf(rsA, goffA[j], ka, sa + (wave * 8 + j) * 1024);
            dma16_buf(rsB, goffB[j], kb, sb + (wave * 8 + j) * 1024);
        }
    };

    // LDS byte offsets of this lane's fragments.
    const int lrow = lane & 31, lk = lane >> 5;
    int offA[4], offB[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int r = wm * 128 + lrow;
        offA[kk] = r * 128 + (((2 * kk + lk) ^ swzK(r)) << 4);
    }
    if constexpr (BCOL) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int r = wn * 128 + lrow;
            offB[kk] = r * 128 + (((2 * kk + lk) ^ swzK(r)) << 4);
        }
    } else {
        const int G = lane >> 4, q = lane & 15;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kr = 8 * (G >> 1) + (q >> 2);
            const int n = wn * 128 + j * 32 + 16 * (G & 1) + 4 * (q & 3);
            offB[j] = kr * 512 + (((n >> 3) ^ swzB(kr)) << 4) + ((n >> 2) & 1) * 8;
        }
    }

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    frag fa[2][4], fb[2][4];
    auto rd = [&](const char *sa, const char *sb, int kk, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            fa[slot][i] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sa + offA[kk] + i * 32 * 128));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (BCOL) {
                fb[slot][j] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(sb + offB[kk] + j * 32 * 128));
            } else {
                const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512));
                const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4 *)to_lds(sb + offB[j] + kk * 16 * 512 + 4 * 512));
                const u32x2 h0 = __builtin_bit_cast(u32x2, t0), h1 = __builtin_bit_cast(u32x2, t1);
                fb[slot][j] = as_frag<frag>(u32x4{h0[0], h0[1], h1[0], h1[1]});
            }
        }
    };
    // swapped operands: acc[i][j] element e is row 32 i + lrow, column
    // 32 j + 8 (e / 4) + 4 lk + e % 4 of the wave's quarter
    auto mm = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::m32(fb[slot][j], fa[slot][i], acc[i][j]);
    };
    // scheduling groups of one k-step: MFMA, LDS read (12 of them: 8 for
    // K-contiguous B), and a DMA instruction after every second MFMA when
    // half a stage's DMA (8 instructions) is issued in this k-step
    constexpr int NRD = BCOL ? 8 : 12;
    auto pattern = [&](bool dma) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (t < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (dma && (t & 1)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
    };
    // Stage s from buffers (sa, sb).  The DMA of a stage goes out in two
    // halves: blocks 0-3 under the last k-step of stage s - 2 (right after
    // the barrier that frees its buffers) and blocks 4-7 under the first
    // k-step of stage s - 1, so no k-step carries more than 8 DMA
    // instructions.  `half2`: issue blocks 4-7 of stage s + 1 into (pa, pb);
    // `next`: wait for this wave's DMA of stage s + 1, meet at the barrier and
    // read stage s + 1's first fragments from (na, nb); `half1`: issue blocks
    // 0-3 of stage s + 2 into this stage's buffers (ra, rb).
    auto stage = [&](int s, const char *sa, const char *sb, const char *na, const char *nb, char *ra, char *rb,
                     char *pa, char *pb, bool half2, bool next, bool half1) __attribute__((always_inline)) {
        if (half2) issue(s + 1, pa, pb, 4, 8);
        rd(sa, sb, 1, 1);
        mm(0);
        pattern(half2);
        __builtin_amdgcn_sched_barrier(0);
        rd(sa, sb, 2, 0);
        mm(1);
        pattern(false);
        __builtin_amdgcn_sched_barrier(0);
        rd(sa, sb, 3, 1);
        mm(0);
        pattern(false);
        __builtin_amdgcn_sched_barrier(0);
        if (next) {
            wait_vmcnt<0>();                         // this wave's DMA of stage s + 1
            __builtin_amdgcn_s_waitcnt(0xc07f);      // and its LDS reads of stage s
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            rd(na, nb, 0, 0);
            if (half1) issue(s + 2, ra, rb, 0, 4);
        }
        mm(1);
        pattern(half1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // nk is even and >= 4: stage 0, pairs of stages, the last three peeled
    // (no conditional DMA inside the loop)
    // A row addend (bias) is loaded with the first stage and kept in LDS as
    // beta * value, so the epilogue does not wait on memory for it.
    const Tout *cin = reinterpret_cast<const Tout *>(a.cin);
    __shared__ __attribute__((aligned(16))) float sRow[256];
    float row_add = 0.f;
    if (c_kind == KUIOPS_C_ROW && n0 + tid < N) row_add = beta * to_f32(cin[n0 + tid]);
    issue(0, sA0, sB0, 0, 8);
    wait_vmcnt<0>();
    sRow[tid] = row_add;      // visible at the epilogue: every stage barrier waits for LDS writes first
    __builtin_amdgcn_s_barrier();
    rd(sA0, sB0, 0, 0);
    issue(1, sA1, sB1, 0, 8);
    stage(0, sA0, sB0, sA1, sB1, sA0, sB0, sA1, sB1, false, true, true);
    int s = 1;
    for (; s + 4 < nk; s += 2) {
        stage(s, sA1, sB1, sA0, sB0, sA1, sB1, sA0, sB0, true, true, true);
        stage(s + 1, sA0, sB0, sA1, sB1, sA0, sB0, sA1, sB1, true, true, true);
    }
    stage(s, sA1, sB1, sA0, sB0, sA1, sB1, sA0, sB0, true, true, true);
    stage(s + 1, sA0, sB0, sA1, sB1, sA0, sB0, sA1, sB1, true, true, false);
    stage(s + 2, sA1, sB1, sA0, sB0, sA1, sB1, sA0, sB0, false, false, false);

    // Epilogue: out = alpha * acc + beta * addend (fp32), one rounding.  The
    // row addend comes from LDS (zeros when there is none); a full-matrix
    // addend (FULLC, its own instance) replaces it.  Branching on the kind
    // inside the kernel costs: per run, 64 scheduling regions (~1.5 us at
    // 4096^3); per kind around the whole epilogue, the compiler hoists the
    // accumulator reads above the branch and spills.
    Tout *out = reinterpret_cast<Tout *>(a.out) + bz * a.stride_o;
    // beta * C[row, col .. col + 3] (8-byte loads where aligned)
    auto addend4 = [&](int64_t row, int64_t col, float v[4]) __attribute__((always_inline)) {
        const Tout *p = cin + row * ldcin + col;
        if (sizeof(Tout) == 2 && col + 3 < N && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
            const u32x2 w = *reinterpret_cast<const u32x2 *>(p);
            const Tout *h = reinterpret_cast<const Tout *>(&w);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = beta * to_f32(h[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = col + e < N ? beta * to_f32(p[e]) : 0.f;
        }
    };
    // the 4 output values of (i, j, g) at tile column cl
    auto value4 = [&](int i, int j, int g, int64_t row, int cl, float v[4]) __attribute__((always_inline)) {
        const f32x4 r4 = *reinterpret_cast<const f32x4 *>(sRow + cl);
        float add[4] = {r4[0], r4[1], r4[2], r4[3]};
        if constexpr (FULLC) {
            if (row < M) addend4(row, n0 + cl, add);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = alpha * acc[i][j][4 * g + e] + add[e];
    };
    if constexpr (sizeof(Tout) == 2) {
        // The tile's image in LDS: rows 64 b .. 64 b + 63 in stage array b,
        // 512 bytes per row, 16-byte chunk c at position c ^ (row & 31).
        auto stg = [&](int b) -> char * { return b == 0 ? sA0 : (b == 1 ? sB0 : (b == 2 ? sA1 : sB1)); };
        const bool fast = vec_store && m0 + 256 <= M && n0 + 256 <= N;
        __builtin_amdgcn_s_barrier();
        // Two halves (accumulator rows i = 0, 1 and then 2, 3): the first
        // half's stores go out while the second half is converted.
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int cl = wn * 128 + j * 32 + 8 * g + 4 * lk;
#pragma unroll
                    for (int i = 2 * h; i < 2 * h + 2; ++i) {
                        const int r = wm * 128 + i * 32 + lrow;
                        float v[4];
                        value4(i, j, g, m0 + r, cl, v);
                        typedef Tout t4 __attribute__((ext_vector_type(4)));
                        t4 w;
#pragma unroll
                        for (int e = 0; e < 4; ++e) w[e] = from_f32<Tout>(v[e]);
                        *reinterpret_cast<u32x2 *>(stg(r >> 6) + (r & 63) * 512 + (((cl >> 3) ^ (r & 31)) << 4) +
                                                   lk * 8) = __builtin_bit_cast(u32x2, w);
                    }
                }
            }
            __syncthreads();
            if (fast) {
                // this half's tile rows: 64 h .. 64 h + 63 of each 128-row band
#pragma unroll
                for (int it = 0; it < 16; ++it) {
                    const int rr = it * 8 + (tid >> 5), ch = tid & 31;
                    const int r = (rr >> 6) * 128 + 64 * h + (rr & 63);
                    const u32x4 v =
                        *reinterpret_cast<const u32x4 *>(stg(r >> 6) + (r & 63) * 512 + ((ch ^ (r & 31)) << 4));
                    // streaming store: the output is not read again here
                    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + (m0 + r) * ldo + n0 + ch * 8));
                }
            }
        }
        if (!fast) {
            for (int it = 0; it < 32; ++it) {
                const int r = it * 8 + (tid >> 5), ch = tid & 31;
                const int64_t grow = m0 + r, gcol = n0 + ch * 8;
                if (grow >= M || gcol >= N) continue;
                const u32x4 v =
                    *reinterpret_cast<const u32x4 *>(stg(r >> 6) + (r & 63) * 512 + ((ch ^ (r & 31)) << 4));
                if (vec_store) {
                    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + grow * ldo + gcol));
                } else {
                    const Tout *e8 = reinterpret_cast<const Tout *>(&v);
                    for (int e = 0; e < 8; ++e)
                        if (gcol + e < N) out[grow * ldo + gcol + e] = e8[e];
                }
            }
        }
    } else {
        // fp32 output: 4 consecutive columns per lane, 16 bytes
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int cl = wn * 128 + j * 32 + 8 * g + 4 * lk;
                const int64_t col = n0 + cl;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t row = m0 + wm * 128 + i * 32 + lrow;
                    float v[4];
                    value4(i, j, g, row, cl, v);
                    if (row >= M) continue;
                    if (vec_store && col + 3 < N) {
                        *reinterpret_cast<f32x4 *>(out + row * ldo + col) = f32x4{v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) out[row * ldo + col + e] = from_f32<Tout>(v[e]);
                    }
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

// KUIOPS_GEMM_KERNEL=dma selects the 8-wave gemm_dma_kernel for the large
// GEMMs (read once per process); the default is gemm_wave_kernel.
static int gemm_kernel_choice() {
    static int choice = -1;
    if (choice < 0) {
        const char *e = getenv("KUIOPS_GEMM_KERNEL");
        choice = (e && e[0] == 'd') ? 1 : 0;
    }
    return choice;
}

static bool dma_eligible(const GemmArgs &a, int64_t batch, bool bcol) {
    // buffer offsets (tile rows x leading dim + K) must stay below 2^31 bytes
    const int64_t lim = (int64_t)1 << 30;
    if ((256 * a.lda + a.K) >= lim) return false;
    if (bcol ? (256 * a.ldb + a.K) >= lim : (a.K * a.ldb + 256) >= lim) return false;
    // batched operands: the addend (addmm only) is not batched
    if (batch > 1 && (a.c_kind != KUIOPS_C_NONE || a.stride_a % 8 || a.stride_b % 8)) return false;
    return a.K % 128 == 0 && a.K > 0 && a.M >= 256 && a.N >= 256 &&
           cdiv(a.M, 256) * cdiv(a.N, 256) * batch >= 128 && cdiv(a.M, 256) * cdiv(a.N, 256) * batch < INT32_MAX;
}

template <typename T, typename Tout>
static int run_mfma(GemmArgs a, int64_t batch, bool bcol, int splits_req, void *ws, size_t ws_bytes,
                    hipStream_t st) {
    if constexpr (sizeof(Tout) == 2) {
        // short K (64 or 128), full 256x256 tiles, several tiles per CU: the
        // persistent kernel overlaps each tile's output stores with the next
        // tile's loads
        const int64_t lim = (int64_t)1 << 30;
        const int64_t total = (a.M / 256) * (a.N / 256) * batch;
        if (splits_req <= 1 && gemm_kernel_choice() != 1 && (a.K == 64 || a.K == 128) &&
            a.c_kind == KUIOPS_C_NONE && a.M % 256 == 0 && a.N % 256 == 0 && 256 * a.lda + a.K < lim &&
            (bcol ? 256 * a.ldb + a.K : a.K * a.ldb + 256) < lim && a.lda % 8 == 0 && a.ldb % 8 == 0 && a.stride_a % 8 == 0 && a.stride_b % 8 == 0 && a.ldo % 8 == 0 &&
            a.stride_o % 8 == 0 && aligned16(a.out) && total >= 2 * (int64_t)num_cus() && total < INT32_MAX) {
            a.tiles_m = (int)(a.M / 256);
            a.tiles_n = (int)(a.N / 256);
            a.vec_store = true;
            const int wgs = (int)min(total, (int64_t)num_cus());
            const dim3 g(wgs), blk(512);
            if (bcol && a.K == 128) hipLaunchKernelGGL((gemm_stream_kernel<T, true, Tout, 2>), g, blk, 0, st, a, (int)total);
            else if (bcol) hipLaunchKernelGGL((gemm_stream_kernel<T, true, Tout, 1>), g, blk, 0, st, a, (int)total);
            else if (a.K == 128) hipLaunchKernelGGL((gemm_stream_kernel<T, false, Tout, 2>), g, blk, 0, st, a, (int)total);
            else hipLaunchKernelGGL((gemm_stream_kernel<T, false, Tout, 1>), g, blk, 0, st, a, (int)total);
            return launch_status();
        }
    }
    if (splits_req <= 1 && dma_eligible(a, batch, bcol)) {
        a.tiles_m = (int)cdiv(a.M, 256);
        a.tiles_n = (int)cdiv(a.N, 256);
        const int vec = sizeof(Tout) == 2 ? 8 : 4;    // elements per vector store
        a.vec_store = a.N % vec == 0 && a.ldo % vec == 0 && a.stride_o % vec == 0 && aligned16(a.out);
        dim3 grid((unsigned)(a.tiles_m * a.tiles_n * batch));
        // 4 waves of 128x128 (one per SIMD, explicit schedule) for deep K;
        // short K loops (bmm's K = 128: two stages, so the prologue and the
        // epilogue dominate) run faster on the 8-wave gemm_dma_kernel, whose
        // second wave per SIMD overlaps them.  KUIOPS_GEMM_KERNEL=dma forces
        // the 8-wave kernel.
        if (gemm_kernel_choice() == 1 || a.K < 512) {
            // Short K is bound by the output stores (bmm 32 x 2048x128x2048
            // writes 268 MB): rasterise row by row so the tiles running
            // together write whole output rows (95 -> 81 us); deep K keeps the
            // grouped order, which shares A / B tiles in each XCD's L2.
            a.raster = a.K < 512 ? 1 : 0;
            a.vec_store = sizeof(Tout) == 2 && a.vec_store;
            if (bcol) hipLaunchKernelGGL((gemm_dma_kernel<T, true, Tout, 2, 4, 64, 2>), grid, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((gemm_dma_kernel<T, false, Tout, 2, 4, 64, 2>), grid, dim3(512), 0, st, a);
        } else {
            const bool full = a.c_kind == KUIOPS_C_FULL;
            if (bcol && full) hipLaunchKernelGGL((gemm_wave_kernel<T, true, Tout, true>), grid, dim3(256), 0, st, a);
            else if (bcol) hipLaunchKernelGGL((gemm_wave_kernel<T, true, Tout, false>), grid, dim3(256), 0, st, a);
            else if (full) hipLaunchKernelGGL((gemm_wave_kernel<T, false, Tout, true>), grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((gemm_wave_kernel<T, false, Tout, false>), grid, dim3(256), 0, st, a);
        }
        return launch_status();
    }
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
