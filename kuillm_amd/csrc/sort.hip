// Sampling-tail ordering and prefix work for gfx950: row sort, row cumsum and
// inverse-CDF multinomial sampling over the last dim (the top-p path of a
// sampler: sort -> softmax -> cumsum -> mask -> scatter -> multinomial).
//
// sort: every element becomes a unique 64-bit key (an order-preserving 32-bit
//   image of the value in the requested direction, then the element index),
//   so sorting keys gives aten's stable sort exactly: ties keep index order,
//   NaN sorts as the largest value.  Pass 1 bitonic-sorts chunks of 2048 keys
//   in LDS (one 1024-thread work-group per chunk); pass 2 gives each key its
//   final rank = its position in its own chunk + the number of smaller keys in
//   every other chunk (a binary search of each other chunk, staged in LDS in
//   turn) and writes value and index there.  For rows of up to 32 chunks the
//   searches run one work-group per (chunk, other chunk) pair and a third
//   pass sums each key's counts and scatters.  Values are copied bit-exactly.
// cumsum: one 1024-thread work-group per row, tiles of 4096 elements (four
//   consecutive per thread, coalesced), block scans plus a running carry
//   (fp32 accumulate for fp32, fp64 for fp64, exact for int64).
// multinomial: with replacement, from caller-supplied uniforms u in [0, 1):
//   sample = the first index whose running weight sum (fp64) exceeds u * total
//   (inverse CDF), so zero-weight entries are never drawn.  One work-group per
//   row.  Rows with a negative, NaN or infinite weight or a zero total set
//   *err_flag and draw index 0.
//
// Semantics: aten.sort / aten.cumsum / aten.multinomial, the reference's
// fallthrough results (no kuiops kernels exist for them: KERNELS.md rows
// "aten.sort.default", "aten.cumsum.default", "aten.multinomial.default").
#include <type_traits>

#include "common.hpp"

namespace kuiops {

constexpr int kSortChunk = 2048;
constexpr int kSortThreads = 1024;
constexpr int kSortPer = kSortChunk / kSortThreads;      // keys per thread

// Unsigned image of v whose order is the value order (NaN above +inf; -0 and
// +0 compare equal, as in aten).
__device__ __forceinline__ uint32_t value_key(float v) {
    const uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
    if (v != v) return 0xffffffffu;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <typename T> __device__ __forceinline__ float sort_val(T v) { return to_f32(v); }

// 64-bit xor shuffle inside a wave (two 32-bit lane swaps).
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

// atomicMin of v into *dst for the whole wave with one LDS atomic (the wave's
// minimum): 1024 same-address atomics serialise.
__device__ __forceinline__ void wave_atomic_min(unsigned long long *dst, uint64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = shfl_xor64(v, off);
        v = o < v ? o : v;
    }
    if ((threadIdx.x & 63) == 0 && v != ~0ull) atomicMin(dst, (unsigned long long)v);
}

// Bitonic sort of the CH keys in s (filled, and the work-group synchronised,
// by the caller; CH / 2 threads), ascending, left in s.  Thread t keeps keys
// 2t and 2t + 1 in registers: stride 1 is an in-thread exchange, strides
// 2..64 pair thread t with thread t ^ (stride / 2) of the same wave (lane
// shuffles, no barrier), and only the stages of stride >= 128 pass through
// LDS (two barriers each; 15 of 66 stages for 2048 keys, against one
// barrier per stage for all of them in LDS).
template <int CH>
__device__ __forceinline__ void bitonic_chunk(uint64_t *s) {
    const int tid = threadIdx.x;
    uint64_t k0 = s[2 * tid], k1 = s[2 * tid + 1];
#pragma unroll
    for (int size = 2; size <= CH; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int pos = 2 * tid;
            const bool up = (pos & size) == 0;
            if (stride == 1) {
                const uint64_t lo = k0 < k1 ? k0 : k1, hi = k0 < k1 ? k1 : k0;
                k0 = up ? lo : hi;
                k1 = up ? hi : lo;
                continue;
            }
            uint64_t p0, p1;
            if (stride <= 64) {
                p0 = shfl_xor64(k0, stride >> 1);
                p1 = shfl_xor64(k1, stride >> 1);
            } else {
                __syncthreads();                     // earlier reads of s are done
                s[pos] = k0;
                s[pos + 1] = k1;
                __syncthreads();
                const int pt = 2 * (tid ^ (stride >> 1));
                p0 = s[pt];
                p1 = s[pt + 1];
            }
            // keys 2t and 2t + 1 share every bit above bit 0
            const bool keep_min = ((pos & stride) == 0) == up;
            k0 = keep_min ? (k0 < p0 ? k0 : p0) : (k0 < p0 ? p0 : k0);
            k1 = keep_min ? (k1 < p1 ? k1 : p1) : (k1 < p1 ? p1 : k1);
        }
    }
    __syncthreads();
    s[2 * tid] = k0;
    s[2 * tid + 1] = k1;
    __syncthreads();
}

// Pass 1: chunk `blockIdx.x` of row `blockIdx.y` -> sorted keys in ws.  With a
// single chunk per row the outputs are written directly.
template <typename T, int CH>
__global__ __launch_bounds__(CH / 2) void sort_chunk_kernel(int64_t n, int nchunks, const T *X, T *vals,
                                                             int64_t *inds, uint64_t *ws, int descending) {
    constexpr int NT = CH / 2;                       // two keys per thread
    __shared__ uint64_t s[CH];
    const int tid = threadIdx.x, c = blockIdx.x;
    const int64_t row = blockIdx.y;
    const T *x = X + row * n;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int p = tid + h * NT;
        const int64_t i = (int64_t)c * CH + p;
        uint64_t key = ~0ull;                        // padding sorts last
        if (i < n) {
            uint32_t k = value_key(sort_val<T>(x[i]));
            if (descending) k = ~k;
            key = ((uint64_t)k << 32) | (uint32_t)i;
        }
        s[p] = key;
    }
    __syncthreads();
    bitonic_chunk<CH>(s);
    if (nchunks == 1) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = tid + h * NT;
            if (p < n) {
                const int64_t src = (int64_t)(uint32_t)s[p];
                vals[row * n + p] = x[src];
                inds[row * n + p] = src;
            }
        }
        return;
    }
    uint64_t *w = ws + (row * nchunks + c) * CH;
#pragma unroll
    for (int h = 0; h < 2; ++h) w[tid + h * NT] = s[tid + h * NT];
}

// Pass 2: rank of each key of chunk blockIdx.x among all keys of the row.
// The other chunks pass through two LDS buffers; the next one is loaded into
// registers while the current one is searched.
template <typename T>
__global__ __launch_bounds__(kSortThreads) void sort_rank_kernel(int64_t n, int nchunks, const T *X, T *vals,
                                                                  int64_t *inds, const uint64_t *ws) {
    __shared__ uint64_t s[2][kSortChunk];
    const int tid = threadIdx.x, c = blockIdx.x;
    const int64_t row = blockIdx.y;
    const uint64_t *base = ws + row * nchunks * (int64_t)kSortChunk;
    uint64_t mine[kSortPer];
    int64_t rank[kSortPer];
#pragma unroll
    for (int h = 0; h < kSortPer; ++h) {
        const int p = tid + h * kSortThreads;
        mine[h] = base[(int64_t)c * kSortChunk + p];
        rank[h] = p;                                 // keys of its own chunk below it
    }
    uint64_t nxt[kSortPer];
    auto load = [&](int o) {
#pragma unroll
        for (int h = 0; h < kSortPer; ++h) nxt[h] = base[(int64_t)o * kSortChunk + tid + h * kSortThreads];
    };
    auto other = [&](int k) { return k < c ? k : k + 1; };   // k-th chunk other than c
    const int nother = nchunks - 1;
    load(other(0));
#pragma unroll
    for (int h = 0; h < kSortPer; ++h) s[0][tid + h * kSortThreads] = nxt[h];
    __syncthreads();
    for (int k = 0; k < nother; ++k) {
        const int cur = k & 1;
        if (k + 1 < nother) load(other(k + 1));
#pragma unroll
        for (int h = 0; h < kSortPer; ++h) {
            // number of keys in the chunk below mine[h] (keys are unique;
            // padding ~0 is above every real key)
            int lo = 0, hi = kSortChunk;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (s[cur][mid] < mine[h]) lo = mid + 1;
                else hi = mid;
            }
            rank[h] += lo;
        }
        if (k + 1 < nother) {
#pragma unroll
            for (int h = 0; h < kSortPer; ++h) s[cur ^ 1][tid + h * kSortThreads] = nxt[h];
        }
        __syncthreads();
    }
    const T *x = X + row * n;
#pragma unroll
    for (int h = 0; h < kSortPer; ++h) {
        if (mine[h] == ~0ull) continue;              // padding
        const int64_t src = (int64_t)(uint32_t)mine[h];
        vals[row * n + rank[h]] = x[src];
        inds[row * n + rank[h]] = src;
    }
}

// Pass 2, wide form (rows of at most kSortWideChunks chunks): one
// work-group per (own chunk c, other chunk o) counts, for every key of
// chunk c, the keys of chunk o below it (a binary search of chunk o staged
// in LDS; o == c: the key's own position), into part[row][o][c][p].  All
// nc^2 searches run at once instead of nc - 1 in turn per work-group.
constexpr int kSortWideChunks = 32;
template <int CH>
__global__ __launch_bounds__(CH / 2) void sort_rank_part_kernel(int nchunks, const uint64_t *ws, uint32_t *part) {
    constexpr int NT = CH / 2;
    __shared__ uint64_t s[CH];
    const int tid = threadIdx.x, c = blockIdx.x, o = blockIdx.y;
    const int64_t row = blockIdx.z;
    const uint64_t *base = ws + row * nchunks * (int64_t)CH;
    uint32_t *out = part + ((row * nchunks + o) * nchunks + c) * (int64_t)CH;
    if (o == c) {
#pragma unroll
        for (int h = 0; h < 2; ++h) out[tid + h * NT] = tid + h * NT;
        return;
    }
    uint64_t mine[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        s[tid + h * NT] = base[(int64_t)o * CH + tid + h * NT];
        mine[h] = base[(int64_t)c * CH + tid + h * NT];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // keys are unique; padding ~0 is above every real key
        int lo = 0, hi = CH;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s[mid] < mine[h]) lo = mid + 1;
            else hi = mid;
        }
        out[tid + h * NT] = (uint32_t)lo;
    }
}

// Pass 3, wide form: each key's rank is the sum of its nc partial counts;
// value and index go there.
template <typename T, int CH>
__global__ __launch_bounds__(CH / 2) void sort_scatter_kernel(int64_t n, int nchunks, const T *X, T *vals,
                                                               int64_t *inds, const uint64_t *ws,
                                                               const uint32_t *part) {
    constexpr int NT = CH / 2;
    const int tid = threadIdx.x, c = blockIdx.x;
    const int64_t row = blockIdx.y;
    const uint64_t *keys = ws + (row * nchunks + c) * (int64_t)CH;
    const T *x = X + row * n;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int p = tid + h * NT;
        const uint64_t key = keys[p];
        if (key == ~0ull) continue;                  // padding
        // (all nc counts load at once: the loop is unrolled to the chunk limit)
        uint32_t rank = 0;
        const uint32_t *pp = part + (row * nchunks * nchunks + c) * (int64_t)CH + p;
#pragma unroll
        for (int o = 0; o < kSortWideChunks; ++o)
            if (o < nchunks) rank += pp[(int64_t)o * nchunks * CH];
        const int64_t src = (int64_t)(uint32_t)key;
        vals[row * n + rank] = x[src];
        inds[row * n + rank] = src;
    }
}

// ------------------------------------------------------------ top-p mask

// The masking step of transformers' TopPLogitsWarper after its sort and
// cumsum, fused: out[sorted_idx[j]] = filter if j < keep_from and the sorted
// cumulative probability cum[j] <= thr, else the sorted value sv[j] (the sort
// copies values bit-exactly, so this is scores[sorted_idx[j]]).  Every
// position of a row is written once (sorted_idx is a permutation): the aten
// sequence le.Scalar, setitem of the kept tail, scatter, masked_fill in one
// pass, spread over the whole grid.
__global__ __launch_bounds__(256) void top_p_mask_kernel(int64_t n, const float *sv, const int64_t *sidx,
                                                          const float *cum, float thr, int64_t keep_from, float fill,
                                                          float *out) {
    const int64_t row = blockIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const int64_t o = row * n + j;
    const int64_t dst = sidx[o];
    if (dst < 0 || dst >= n) return;                 // not a permutation of the row: no stray store
    out[row * n + dst] = (j < keep_from && cum[o] <= thr) ? fill : sv[o];
}

// ------------------------------------------------------------------ scans

template <typename A>
__device__ __forceinline__ A wave_incl_scan(A x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const A y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    return x;
}

// Exclusive block scan of one value per thread (1024 threads), fixed order;
// returns the exclusive prefix and the block total.
template <typename A>
__device__ __forceinline__ A block_scan_excl(A v, A *s_wave, A &total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const A incl = wave_incl_scan(v, lane);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const A w = lane < kSortThreads / 64 ? s_wave[lane] : A(0);
        const A ws = wave_incl_scan(w, lane);
        if (lane < kSortThreads / 64) s_wave[lane] = ws - w;
        if (lane == kSortThreads / 64 - 1) s_wave[kSortThreads / 64] = ws;
    }
    __syncthreads();
    const A excl = s_wave[wave] + (incl - v);
    total = s_wave[kSortThreads / 64];
    __syncthreads();
    return excl;
}

// Rows are scanned in tiles of 1024 x 4 consecutive elements: thread t loads
// elements 4t..4t+3 of the tile (coalesced), scans them in registers, and a
// block scan of the per-thread sums plus the carry of the earlier tiles
// offsets them.
constexpr int kScanVPT = 4;
constexpr int kScanTile = kSortThreads * kScanVPT;

// Loads the run x[b .. b + RP) into v (zeros past n): 16-byte loads when the
// run is whole and aligned, else element by element.
template <typename T, typename A, int RP>
__device__ __forceinline__ void load_run(const T *x, int64_t b, int64_t n, A *v) {
    constexpr int E = 16 / sizeof(T);           // elements per 16-byte load
    if (RP % E == 0 && b + RP <= n && ((reinterpret_cast<uintptr_t>(x + b) & 15) == 0)) {
#pragma unroll
        for (int c = 0; c < RP / E; ++c) {
            const u32x4 raw = *reinterpret_cast<const u32x4 *>(x + b + c * E);
            typedef T tv __attribute__((ext_vector_type(E)));
            const tv t = __builtin_bit_cast(tv, raw);
#pragma unroll
            for (int e = 0; e < E; ++e) v[c * E + e] = (A)t[e];
        }
    } else {
#pragma unroll
        for (int j = 0; j < RP; ++j) v[j] = b + j < n ? (A)x[b + j] : A(0);
    }
}

// Stores y[b + j] = v[j] + off for the run (16-byte stores when whole and aligned).
template <typename T, typename A, int RP>
__device__ __forceinline__ void store_run(T *y, int64_t b, int64_t n, const A *v, A off) {
    constexpr int E = 16 / sizeof(T);
    if (RP % E == 0 && b + RP <= n && ((reinterpret_cast<uintptr_t>(y + b) & 15) == 0)) {
#pragma unroll
        for (int c = 0; c < RP / E; ++c) {
            typedef T tv __attribute__((ext_vector_type(E)));
            tv t;
#pragma unroll
            for (int e = 0; e < E; ++e) t[e] = (T)(off + v[c * E + e]);
            *reinterpret_cast<u32x4 *>(y + b + c * E) = __builtin_bit_cast(u32x4, t);
        }
    } else {
#pragma unroll
        for (int j = 0; j < RP; ++j)
            if (b + j < n) y[b + j] = (T)(off + v[j]);
    }
}

// Rows of 8K..32K elements through LDS: coalesced 16-byte loads (lane q takes
// elements E q .. E q + E - 1, E per 16 bytes) into a [1024][33] float array,
// then each thread reads its 32-element run at the 33-float pitch (bank
// conflict free).  Loading the runs straight from memory touches 64 cache
// lines per load instruction (a 128-byte lane stride), which the texture
// path serves one line at a time.  Elements past n read as 0.
constexpr int kStageRP = 32, kStagePitch = 33;
template <typename T>
__device__ __forceinline__ void stage_row_in(const T *x, int64_t n, float *sm, float *v) {
    constexpr int E = 16 / sizeof(T);
    constexpr int Q = kSortThreads * kStageRP / E;              // 16-byte chunks of a full row
    const int tid = threadIdx.x;
    const bool vec = n % E == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
#pragma unroll
    for (int k = 0; k < Q / kSortThreads; ++k) {
        const int q = k * kSortThreads + tid, e0 = q * E;
        float t[E];
        if (vec && e0 + E <= n) {
            typedef T tv __attribute__((ext_vector_type(E)));
            const tv r = __builtin_bit_cast(tv, *reinterpret_cast<const u32x4 *>(x + e0));
#pragma unroll
            for (int e = 0; e < E; ++e) t[e] = to_f32(r[e]);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) t[e] = e0 + e < n ? to_f32(x[e0 + e]) : 0.f;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) sm[((e0 + e) >> 5) * kStagePitch + ((e0 + e) & 31)] = t[e];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kStageRP; ++j) v[j] = sm[tid * kStagePitch + j];
}

// fp32 cumsum of rows of 8K..32K elements: the row comes in through LDS
// (stage_row_in), each run is scanned in registers and offset by one block
// scan, and the result goes out through LDS as coalesced 16-byte stores.
__global__ __launch_bounds__(kSortThreads) void cumsum_stage_kernel(int64_t n, const float *X, float *Y) {
    __shared__ float sm[kSortThreads * kStagePitch];
    __shared__ float s_wave[kSortThreads / 64 + 1];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const float *x = X + row * n;
    float *y = Y + row * n;
    float v[kStageRP];
    stage_row_in<float>(x, n, sm, v);
#pragma unroll
    for (int j = 1; j < kStageRP; ++j) v[j] += v[j - 1];
    float total;
    const float excl = block_scan_excl<float>(v[kStageRP - 1], s_wave, total);   // (ends with a barrier)
#pragma unroll
    for (int j = 0; j < kStageRP; ++j) sm[tid * kStagePitch + j] = excl + v[j];
    __syncthreads();
    const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
    for (int k = 0; k < kStageRP / 4; ++k) {
        const int e0 = (k * kSortThreads + tid) * 4;
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = sm[((e0 + e) >> 5) * kStagePitch + ((e0 + e) & 31)];
        if (vec && e0 + 4 <= n) {
            *reinterpret_cast<f32x4 *>(y + e0) = f32x4{t[0], t[1], t[2], t[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (e0 + e < n) y[e0 + e] = t[e];
        }
    }
}

// Rows of at most 1024 x RP elements: thread t owns the contiguous run
// [RP t, RP t + RP), loaded at once (every cache line is used whole by its
// lane), scanned in registers, offset by one block scan.
template <typename T, int RP>
__global__ __launch_bounds__(kSortThreads) void cumsum_reg_kernel(int64_t n, const T *X, T *Y) {
    typedef T A;
    __shared__ A s_wave[kSortThreads / 64 + 1];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const T *x = X + row * n;
    T *y = Y + row * n;
    const int64_t b = (int64_t)tid * RP;
    A v[RP];
    load_run<T, A, RP>(x, b, n, v);
#pragma unroll
    for (int j = 1; j < RP; ++j) v[j] += v[j - 1];
    A total;
    const A excl = block_scan_excl<A>(v[RP - 1], s_wave, total);
    store_run<T, A, RP>(y, b, n, v, excl);
}

template <typename T>
__global__ __launch_bounds__(kSortThreads) void cumsum_kernel(int64_t n, const T *X, T *Y) {
    typedef T A;                                // fp32 accumulate for fp32, fp64 / int64 exact types
    __shared__ A s_wave[kSortThreads / 64 + 1];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const T *x = X + row * n;
    T *y = Y + row * n;
    A carry = A(0);
    for (int64_t t0 = 0; t0 < n; t0 += kScanTile) {
        const int64_t b = t0 + (int64_t)tid * kScanVPT;
        A v[kScanVPT];
#pragma unroll
        for (int j = 0; j < kScanVPT; ++j) v[j] = b + j < n ? (A)x[b + j] : A(0);
#pragma unroll
        for (int j = 1; j < kScanVPT; ++j) v[j] += v[j - 1];
        A total;
        const A excl = block_scan_excl<A>(v[kScanVPT - 1], s_wave, total) + carry;
#pragma unroll
        for (int j = 0; j < kScanVPT; ++j)
            if (b + j < n) y[b + j] = (T)(excl + v[j]);
        carry += total;
    }
}

// ------------------------------------------------------------ multinomial

// Pass 1 sums the row (fp64) and validates it; pass 2 walks the tiles with a
// running fp64 prefix per sample: the first element whose inclusive prefix
// exceeds u * total (and whose weight is positive) is the draw, found as the
// smallest such index of the tile (LDS atomic min).
template <typename T>
__global__ __launch_bounds__(kSortThreads) void multinomial_kernel(int64_t n, int64_t ns, const T *P, const float *U,
                                                                    int64_t *out, int *err) {
    __shared__ double s_wave[kSortThreads / 64 + 1];
    __shared__ int s_bad;
    __shared__ unsigned long long s_pick;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const T *p = P + row * n;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    double sum = 0.0;
    int64_t last_pos = -1;
    bool bad = false;
    for (int64_t t0 = 0; t0 < n; t0 += kScanTile) {
        const int64_t b = t0 + (int64_t)tid * kScanVPT;
#pragma unroll
        for (int j = 0; j < kScanVPT; ++j) {
            if (b + j >= n) continue;
            const double v = (double)to_f32_or_self(p[b + j]);
            if (!(v >= 0.0) || v == INFINITY) bad = true;      // negative, NaN, inf
            if (v > 0.0) last_pos = b + j;
            sum += v;
        }
    }
    if (bad) s_bad = 1;
    double total;
    (void)block_scan_excl<double>(sum, s_wave, total);
    if (tid == 0) s_pick = 0ull;
    __syncthreads();
    // the last positive weight of the row: draws whose target the rounded
    // prefix sums never exceed (u rounding onto the total) take it
    {
        uint64_t lp = (uint64_t)(last_pos + 1);      // 0: none; one atomic per wave
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint64_t o = shfl_xor64(lp, off);
            lp = o > lp ? o : lp;
        }
        if ((tid & 63) == 0 && lp > 0) atomicMax(&s_pick, (unsigned long long)(lp - 1));
    }
    __syncthreads();
    const int64_t row_last = (int64_t)s_pick;
    const bool row_bad = s_bad != 0 || !(total > 0.0);
    for (int64_t sidx = 0; sidx < ns; ++sidx) {
        if (row_bad) {
            if (tid == 0) {
                out[row * ns + sidx] = 0;
                if (err) *err = 1;
            }
            continue;
        }
        const double target = (double)U[row * ns + sidx] * total;
        double carry = 0.0;
        int64_t pick = -1;
        for (int64_t t0 = 0; t0 < n && pick < 0; t0 += kScanTile) {
            const int64_t b = t0 + (int64_t)tid * kScanVPT;
            double v[kScanVPT], c[kScanVPT];
#pragma unroll
            for (int j = 0; j < kScanVPT; ++j) v[j] = b + j < n ? (double)to_f32_or_self(p[b + j]) : 0.0;
            c[0] = v[0];
#pragma unroll
            for (int j = 1; j < kScanVPT; ++j) c[j] = c[j - 1] + v[j];
            double tile_total;
            const double excl = block_scan_excl<double>(c[kScanVPT - 1], s_wave, tile_total) + carry;
            if (tid == 0) s_pick = ~0ull;
            __syncthreads();
            uint64_t cand = ~0ull;                   // this thread's first qualifying index
#pragma unroll
            for (int j = kScanVPT - 1; j >= 0; --j)
                if (b + j < n && v[j] > 0.0 && excl + c[j] > target) cand = (uint64_t)(b + j);
            wave_atomic_min(&s_pick, cand);
            __syncthreads();
            if (s_pick != ~0ull) pick = (int64_t)s_pick;
            carry += tile_total;
            __syncthreads();
        }
        if (tid == 0) out[row * ns + sidx] = pick >= 0 ? pick : row_last;
    }
}

// Rows of at most 1024 x RP weights: thread t holds the contiguous run
// [RP t, RP t + RP) in registers; one block scan gives each run its fp64
// prefix, and each draw is the smallest index (LDS atomic min) whose
// inclusive prefix exceeds u * total with a positive weight.
template <typename T, int RP>
__global__ __launch_bounds__(kSortThreads) void multinomial_reg_kernel(int64_t n, int64_t ns, const T *P,
                                                                        const float *U, int64_t *out, int *err) {
    __shared__ double s_wave[kSortThreads / 64 + 1];
    __shared__ int s_bad;
    __shared__ unsigned long long s_pick, s_last;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    static_assert(RP == kStageRP, "staged run length");
    __shared__ float sm[kSortThreads * kStagePitch];
    const T *p = P + row * n;
    const int64_t b = (int64_t)tid * RP;
    if (tid == 0) { s_bad = 0; s_last = 0ull; }
    float v[RP];
    stage_row_in<T>(p, n, sm, v);
    double sum = 0.0;
    int64_t last_pos = -1;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < RP; ++j) {
        if (!(v[j] >= 0.f) || v[j] == INFINITY) bad = true;     // negative, NaN, inf
        if (v[j] > 0.f) last_pos = b + j;
        sum += (double)v[j];
    }
    // the row's last positive weight: a wave maximum, then one LDS atomic per
    // wave (1024 same-address atomics serialise: ~5 us)
    uint64_t lp = (uint64_t)(last_pos + 1);          // 0: none
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = shfl_xor64(lp, off);
        lp = o > lp ? o : lp;
    }
    __syncthreads();
    if (bad) s_bad = 1;
    if ((tid & 63) == 0 && lp > 0) atomicMax(&s_last, (unsigned long long)(lp - 1));
    double total;
    const double excl = block_scan_excl<double>(sum, s_wave, total);
    const bool row_bad = s_bad != 0 || !(total > 0.0);
    const int64_t row_last = (int64_t)s_last;
    for (int64_t sidx = 0; sidx < ns; ++sidx) {
        if (row_bad) {
            if (tid == 0) {
                out[row * ns + sidx] = 0;
                if (err) *err = 1;
            }
            continue;
        }
        const double target = (double)U[row * ns + sidx] * total;
        if (tid == 0) s_pick = ~0ull;
        __syncthreads();
        uint64_t cand = ~0ull;                       // this thread's first qualifying index
        if (excl + sum > target) {
            double run = excl;
#pragma unroll
            for (int j = 0; j < RP; ++j) {
                run += (double)v[j];
                if (run > target && v[j] > 0.f) {
                    cand = (uint64_t)(b + j);
                    break;
                }
            }
        }
        wave_atomic_min(&s_pick, cand);
        __syncthreads();
        if (tid == 0) out[row * ns + sidx] = s_pick != ~0ull ? (int64_t)s_pick : row_last;
        __syncthreads();
    }
}

// The wide rank form while its partial counts stay small (m * nc^2 chunks of
// counts: at most 64 MiB of 1024-key chunks, 128 MiB of 2048-key ones).
static bool sort_wide(int64_t m, int64_t nc) { return nc > 1 && nc <= kSortWideChunks && m * nc * nc <= 16384; }

// Keys per chunk: 1024 (512 threads; the bitonic pass is about half as
// long) whenever the wide rank form takes the row at that size, else 2048.
static int sort_chunk_for(int64_t m, int64_t n) {
    const int64_t nc = cdiv(n, 1024);
    return nc <= 1 || sort_wide(m, nc) ? 1024 : kSortChunk;
}

// keys, plus the partial counts of the wide form
size_t sort_workspace_bytes(int64_t m, int64_t n) {
    const int ch = sort_chunk_for(m, n);
    const int64_t nc = cdiv(n, ch);
    if (nc <= 1) return 0;
    size_t bytes = (size_t)m * nc * ch * sizeof(uint64_t);
    if (sort_wide(m, nc)) bytes += (size_t)m * nc * nc * ch * sizeof(uint32_t);
    return bytes;
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_sort_lastdim(int64_t m, int64_t n, int dtype, const void *X, void *values, int64_t *indices,
                                   int descending, void *workspace, size_t workspace_bytes, void *stream) {
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!X || !values || !indices) return KUIOPS_E_INVALID;
    if (n >= (int64_t)UINT32_MAX || m > 65535) return KUIOPS_E_UNSUPPORTED;
    const int ch = sort_chunk_for(m, n);
    const int64_t nc64 = cdiv(n, ch);
    if (nc64 > 65535) return KUIOPS_E_UNSUPPORTED;
    const int nc = (int)nc64;
    const size_t need = sort_workspace_bytes(m, n);
    if (need && (!workspace || workspace_bytes < need)) return KUIOPS_E_WORKSPACE;
    uint64_t *ws = reinterpret_cast<uint64_t *>(workspace);
    const bool wide = sort_wide(m, nc);
    uint32_t *part = wide ? reinterpret_cast<uint32_t *>(ws + (size_t)m * nc * ch) : nullptr;
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)nc, (unsigned)m);
    const dim3 pairs((unsigned)nc, (unsigned)nc, (unsigned)m);
#define KUIOPS_SORT_CH(T, CH)                                                                                 \
    do {                                                                                                      \
        hipLaunchKernelGGL((sort_chunk_kernel<T, CH>), grid, dim3(CH / 2), 0, st, n, nc, (const T *)X,       \
                           (T *)values, indices, ws, descending);                                              \
        if (wide) {                                                                                           \
            hipLaunchKernelGGL((sort_rank_part_kernel<CH>), pairs, dim3(CH / 2), 0, st, nc,                   \
                               (const uint64_t *)ws, part);                                                   \
            hipLaunchKernelGGL((sort_scatter_kernel<T, CH>), grid, dim3(CH / 2), 0, st, n, nc, (const T *)X,  \
                               (T *)values, indices, (const uint64_t *)ws, (const uint32_t *)part);          \
        } else if (nc > 1) {                                                                                  \
            hipLaunchKernelGGL(sort_rank_kernel<T>, grid, dim3(kSortThreads), 0, st, n, nc, (const T *)X,     \
                               (T *)values, indices, (const uint64_t *)ws);                                   \
        }                                                                                                     \
    } while (0)
#define KUIOPS_SORT(T)                                                                                        \
    do {                                                                                                      \
        if (ch == 1024) KUIOPS_SORT_CH(T, 1024);                                                              \
        else KUIOPS_SORT_CH(T, 2048);                                                                         \
    } while (0)
    switch (dtype) {
        case KUIOPS_F32: KUIOPS_SORT(float); break;
        case KUIOPS_BF16: KUIOPS_SORT(bf16_t); break;
        case KUIOPS_F16: KUIOPS_SORT(f16_t); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
#undef KUIOPS_SORT
#undef KUIOPS_SORT_CH
    return launch_status();
}

extern "C" int kuiops_top_p_mask(int64_t m, int64_t n, const float *sorted_vals, const int64_t *sorted_idx,
                                 const float *cum, double top_p, int64_t min_keep, double filter_value, float *out,
                                 void *stream) {
    if (m < 0 || n < 0 || min_keep < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!sorted_vals || !sorted_idx || !cum || !out) return KUIOPS_E_INVALID;
    if (m > 65535 || cdiv(n, 256) > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    // thr: the Python float 1 - top_p, compared with fp32 probabilities in fp32;
    // remove[..., -min_keep:] = False keeps the last min_keep sorted positions
    // (all of them for min_keep == 0, as Python's [-0:] slice does)
    const float thr = (float)(1.0 - top_p);
    const int64_t keep_from = min_keep == 0 ? 0 : (min_keep >= n ? 0 : n - min_keep);
    hipLaunchKernelGGL(top_p_mask_kernel, dim3((unsigned)cdiv(n, 256), (unsigned)m), dim3(256), 0, as_stream(stream),
                       n, sorted_vals, sorted_idx, cum, thr, keep_from, (float)filter_value, out);
    return launch_status();
}

extern "C" int kuiops_cumsum_lastdim(int64_t m, int64_t n, int dtype, const void *X, void *Y, void *stream) {
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!X || !Y) return KUIOPS_E_INVALID;
    if (m > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)m);
#define KUIOPS_CUMSUM(T)                                                                                      \
    do {                                                                                                      \
        if (n <= kSortThreads * 8)                                                                            \
            hipLaunchKernelGGL((cumsum_reg_kernel<T, 8>), grid, dim3(kSortThreads), 0, st, n, (const T *)X, (T *)Y); \
        else if (n <= kSortThreads * 32 && std::is_same<T, float>::value)                                     \
            hipLaunchKernelGGL(cumsum_stage_kernel, grid, dim3(kSortThreads), 0, st, n, (const float *)X,     \
                               (float *)Y);                                                                   \
        else if (n <= kSortThreads * 32)                                                                      \
            hipLaunchKernelGGL((cumsum_reg_kernel<T, 32>), grid, dim3(kSortThreads), 0, st, n, (const T *)X, (T *)Y); \
        else                                                                                                  \
            hipLaunchKernelGGL(cumsum_kernel<T>, grid, dim3(kSortThreads), 0, st, n, (const T *)X, (T *)Y);   \
    } while (0)
    switch (dtype) {
        case KUIOPS_F32: KUIOPS_CUMSUM(float); break;
        case KUIOPS_F64: KUIOPS_CUMSUM(double); break;
        case KUIOPS_I64: KUIOPS_CUMSUM(int64_t); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
#undef KUIOPS_CUMSUM
    return launch_status();
}

extern "C" int kuiops_multinomial(int64_t m, int64_t n, int dtype, const void *probs, int64_t num_samples,
                                  const float *uniforms, int64_t *out, int *err_flag, void *stream) {
    if (m < 0 || n < 0 || num_samples < 0) return KUIOPS_E_INVALID;
    if (m == 0 || num_samples == 0) return KUIOPS_OK;
    if (n == 0 || !probs || !uniforms || !out) return KUIOPS_E_INVALID;
    if (m > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)m);
    if (n <= kSortThreads * 32 && dtype != KUIOPS_F64) {
        switch (dtype) {
            case KUIOPS_F32: hipLaunchKernelGGL((multinomial_reg_kernel<float, 32>), grid, dim3(kSortThreads), 0, st, n, num_samples, (const float *)probs, uniforms, out, err_flag); break;
            case KUIOPS_BF16: hipLaunchKernelGGL((multinomial_reg_kernel<bf16_t, 32>), grid, dim3(kSortThreads), 0, st, n, num_samples, (const bf16_t *)probs, uniforms, out, err_flag); break;
            case KUIOPS_F16: hipLaunchKernelGGL((multinomial_reg_kernel<f16_t, 32>), grid, dim3(kSortThreads), 0, st, n, num_samples, (const f16_t *)probs, uniforms, out, err_flag); break;
            default: return KUIOPS_E_UNSUPPORTED;
        }
        return launch_status();
    }
    switch (dtype) {
        case KUIOPS_F32: hipLaunchKernelGGL(multinomial_kernel<float>, grid, dim3(kSortThreads), 0, st, n, num_samples, (const float *)probs, uniforms, out, err_flag); break;
        case KUIOPS_F64: hipLaunchKernelGGL(multinomial_kernel<double>, grid, dim3(kSortThreads), 0, st, n, num_samples, (const double *)probs, uniforms, out, err_flag); break;
        case KUIOPS_BF16: hipLaunchKernelGGL(multinomial_kernel<bf16_t>, grid, dim3(kSortThreads), 0, st, n, num_samples, (const bf16_t *)probs, uniforms, out, err_flag); break;
        case KUIOPS_F16: hipLaunchKernelGGL(multinomial_kernel<f16_t>, grid, dim3(kSortThreads), 0, st, n, num_samples, (const f16_t *)probs, uniforms, out, err_flag); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}
