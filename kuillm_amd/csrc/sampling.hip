// Sampling tail for gfx950: row softmax and row top-k over the last dim.
//
// softmax_kernel: one work-group per row; pass 1 keeps a per-thread online
// (max, sum) pair, merged across the wave with shuffles and across waves in
// LDS in a fixed order; pass 2 writes exp(x - max) / sum.  fp32 math (fp64 for
// f64 input).  Semantics: aten._softmax (kuipy/kuiops.py:578-610,
// tests/test_jit_ops.py:141-155).
//
// topk: one 1024-thread work-group per row.  Values are mapped to 32-bit keys
// whose unsigned order is the requested order (NaN above +inf, as aten.topk
// treats it).  k = 1 is a single arg-max pass.  Otherwise an MSB-first radix
// select (4 passes of 8 bits, LDS histograms) finds the k-th key; the selected
// elements are gathered in index order with block prefix sums (so ties at the
// k-th place keep the lowest indices) and then bitonic-sorted in LDS by
// (key descending, index ascending).  Values are copied bit-exactly.
// There is no reference kernel (kuiops/topk/.gitkeep); aten.topk is the
// reference's result.
#include "top1.hpp"

namespace kuiops {

// --------------------------------------------------------------- softmax

template <typename T> struct AccT { typedef float type; };
template <> struct AccT<double> { typedef double type; };


template <typename A>
__device__ __forceinline__ void sm_merge(A &m, A &s, A m2, A s2) {
    const A M = m > m2 ? m : m2;
    if (M == -(A)INFINITY) return;            // both empty
    s = s * acc_exp(m - M) + s2 * acc_exp(m2 - M);
    m = M;
}

// Rows of at most 1024 elements: one wave per row, 4 rows per work-group,
// the row held in registers (16 values per lane); one read, one write.
template <typename T>
__global__ __launch_bounds__(256) void softmax_wave_kernel(int64_t m, int64_t n, const T *X, T *Y) {
    typedef typename AccT<T>::type A;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const T *x = X + row * n;
    T *y = Y + row * n;
    A v[16];
    A mx = -(A)INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int64_t i = lane + 64 * j;
        v[j] = i < n ? (A)to_f32_or_self(x[i]) : -(A)INFINITY;
        mx = v[j] > mx ? v[j] : mx;
    }
    // a NaN never wins `>`: carry it into the max explicitly so the row is NaN
#pragma unroll
    for (int j = 0; j < 16; ++j) if (v[j] != v[j]) mx = v[j];
    mx = wave_max(mx);
    A sum = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        v[j] = acc_exp(v[j] - mx);
        if (lane + 64 * j < n) sum += v[j];
    }
    sum = wave_sum(sum);
    const A inv = (A)1 / sum;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int64_t i = lane + 64 * j;
        if (i < n) y[i] = (T)(v[j] * inv);
    }
}

// Longer rows: one 1024-thread work-group per row.  Rows of at most
// 32 * 1024 elements stay in registers (one read); longer rows use an online
// (max, sum) pass and a second read.

template <typename T>
__global__ __launch_bounds__(kSmThreads) void softmax_row_kernel(int64_t n, const T *X, T *Y) {
    typedef typename AccT<T>::type A;
    const int64_t row = blockIdx.x;
    const T *x = X + row * n;
    T *y = Y + row * n;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ A s_a[kSmThreads / 64], s_b[kSmThreads / 64];
    const bool cached = n <= (int64_t)kSmThreads * kSmCache;
    A v[kSmCache];
    A m = -(A)INFINITY, s = 0;
    if (cached) {
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int64_t i = tid + (int64_t)kSmThreads * j;
            v[j] = i < n ? (A)to_f32_or_self(x[i]) : -(A)INFINITY;
            m = (v[j] > m || v[j] != v[j]) ? v[j] : m;
        }
        m = wave_max(m);
        if (lane == 0) s_a[wave] = m;
        __syncthreads();
        m = s_a[0];
#pragma unroll
        for (int w = 1; w < kSmThreads / 64; ++w) m = (s_a[w] > m || s_a[w] != s_a[w]) ? s_a[w] : m;
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            v[j] = acc_exp(v[j] - m);
            if (tid + (int64_t)kSmThreads * j < n) s += v[j];
        }
        s = wave_sum(s);
        if (lane == 0) s_b[wave] = s;
        __syncthreads();
        s = 0;
#pragma unroll
        for (int w = 0; w < kSmThreads / 64; ++w) s += s_b[w];
        const A inv = (A)1 / s;
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int64_t i = tid + (int64_t)kSmThreads * j;
            if (i < n) y[i] = (T)(v[j] * inv);
        }
        return;
    }
    for (int64_t i = tid; i < n; i += kSmThreads) {
        const A e = (A)to_f32_or_self(x[i]);
        if (e > m) {
            s = (m == -(A)INFINITY ? (A)0 : s * acc_exp(m - e)) + (A)1;
            m = e;
        } else if (e != -(A)INFINITY) {
            s += acc_exp(e - m);     // NaN propagates into s
        }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const A m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
        if (lane & off) { A mm = m2, ss = s2; sm_merge(mm, ss, m, s); m = mm; s = ss; }
        else sm_merge(m, s, m2, s2);
    }
    if (lane == 0) { s_a[wave] = m; s_b[wave] = s; }
    __syncthreads();
    A M = s_a[0], S = s_b[0];
#pragma unroll
    for (int w = 1; w < kSmThreads / 64; ++w) sm_merge(M, S, s_a[w], s_b[w]);
    const A inv = (A)1 / S;
    for (int64_t i = tid; i < n; i += kSmThreads) {
        const A e = (A)to_f32_or_self(x[i]);
        y[i] = (T)(acc_exp(e - M) * inv);
    }
}

// ------------------------------------------------------------------ topk


template <typename T> __device__ __forceinline__ float load_f(const T *p) { return to_f32(*p); }

constexpr int kTopkThreads = 1024;
constexpr int kTopkMaxK = 1024;

// Block-wide exclusive prefix sum of one int per thread (1024 threads).
__device__ __forceinline__ int block_excl_scan(int v, int *s_warp, int &total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_warp[wave] = x;
    __syncthreads();
    if (wave == 0) {
        int w = lane < kTopkThreads / 64 ? s_warp[lane] : 0;
        int ws = w;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(ws, off, 64);
            if (lane >= off) ws += y;
        }
        if (lane < kTopkThreads / 64) s_warp[lane] = ws - w;   // exclusive per wave
        if (lane == kTopkThreads / 64 - 1) s_warp[kTopkThreads / 64] = ws;
    }
    __syncthreads();
    const int excl = s_warp[wave] + x - v;
    total = s_warp[kTopkThreads / 64];
    __syncthreads();
    return excl;
}

// The largest key T such that at least `k` of the participating threads'
// values are >= T (the k-th largest), by a 4-pass MSB radix select over one
// value per thread.  Threads with part == false take no part.
__device__ uint32_t block_kth_largest(uint32_t v, bool part, int k, int *hist, uint32_t *s_state) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) { s_state[0] = 0; s_state[1] = 0; s_state[2] = (uint32_t)k; }
    __syncthreads();
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_state[0], mask = s_state[1];
        if (part && (v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255], 1);
        __syncthreads();
        if (wave == 0) {
            const int rem = (int)s_state[2];
            int c[4], cs = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) { c[j] = hist[255 - (lane * 4 + j)]; cs += c[j]; }
            int incl = cs;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int y = __shfl_up(incl, off, 64);
                if (lane >= off) incl += y;
            }
            int before = incl - cs;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (before < rem && before + c[j] >= rem) {
                    const uint32_t d = 255 - (lane * 4 + j);
                    s_state[0] = prefix | (d << shift);
                    s_state[1] = mask | (255u << shift);
                    s_state[2] = (uint32_t)(rem - before);
                }
                before += c[j];
            }
        }
        __syncthreads();
    }
    const uint32_t t = s_state[0];
    __syncthreads();
    return t;
}

// Descending bitonic sort of 128 keys held two per lane by one wave (lane l:
// positions 2l, 2l + 1): stride 1 in-lane, strides 2..64 by lane shuffles,
// no barriers.
__device__ __forceinline__ uint64_t topk_shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, 64), hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void wave_bitonic128_desc(uint64_t &k0, uint64_t &k1) {
    const int pos = 2 * (threadIdx.x & 63);
#pragma unroll
    for (int size = 2; size <= 128; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const bool desc = (pos & size) == 0;
            if (stride == 1) {
                const uint64_t hi = k0 > k1 ? k0 : k1, lo = k0 > k1 ? k1 : k0;
                k0 = desc ? hi : lo;
                k1 = desc ? lo : hi;
                continue;
            }
            const uint64_t p0 = topk_shfl_xor64(k0, stride >> 1), p1 = topk_shfl_xor64(k1, stride >> 1);
            const bool keep_max = ((pos & stride) == 0) == desc;
            k0 = keep_max ? (k0 > p0 ? k0 : p0) : (k0 > p0 ? p0 : k0);
            k1 = keep_max ? (k1 > p1 ? k1 : p1) : (k1 > p1 ? p1 : k1);
        }
    }
}

constexpr int kTopkFastPer = 32;       // keys per thread held in registers (n <= 32768)
constexpr int kTopkFastMaxK = 512;
constexpr int kTopkCandCap = 2048;     // candidates the fast path sorts

template <typename T>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(int64_t n, int k, const T *X, T *vals,
                                                            int64_t *inds, int largest) {
    const int64_t row = blockIdx.x;
    const T *x = X + row * n;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool lg = largest != 0;

    if (k == 1) {
        // arg-max with lowest-index tie break: composite (key, ~index) maximum.
        uint64_t best = 0;
        // (unrolled: eight loads in flight per thread)
#pragma unroll 8
        for (int64_t i = tid; i < n; i += kTopkThreads) {
            const uint64_t c = ((uint64_t)order_key(load_f(x + i), lg) << 32) | (uint32_t)~(uint32_t)i;
            best = c > best ? c : best;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint64_t o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        __shared__ uint64_t s_best[kTopkThreads / 64];
        if (lane == 0) s_best[wave] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = s_best[0];
            for (int w = 1; w < kTopkThreads / 64; ++w) b = s_best[w] > b ? s_best[w] : b;
            const int64_t idx = (int64_t)(uint32_t)~(uint32_t)(b & 0xffffffffu);
            vals[row] = x[idx];
            inds[row] = idx;
        }
        return;
    }

    __shared__ int hist[256];
    __shared__ int s_scan[kTopkThreads / 64 + 1];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remaining;
    __shared__ uint64_t s_sel[kTopkMaxK];

    if (n <= (int64_t)kTopkThreads * kTopkFastPer && k <= kTopkFastMaxK) {
        // Fast path: the row stays in registers (element j * 1024 + tid).
        // T = the k-th largest of the per-thread maxima bounds the top k from
        // below (k threads hold a key >= T), and usually few keys reach it:
        // those candidates are gathered with one block scan and sorted.
        __shared__ uint64_t s_cand[kTopkCandCap];
        __shared__ uint32_t s_state[3];
        uint32_t key[kTopkFastPer];
        uint32_t mx = 0;
        bool has = false;
#pragma unroll
        for (int j = 0; j < kTopkFastPer; ++j) {
            const int64_t i = (int64_t)j * kTopkThreads + tid;
            key[j] = i < n ? order_key(load_f(x + i), lg) : 0u;
            if (i < n) { mx = has ? max(mx, key[j]) : key[j]; has = true; }
        }
        const uint32_t thr = block_kth_largest(mx, has, k, hist, s_state);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kTopkFastPer; ++j) cnt += ((int64_t)j * kTopkThreads + tid < n) && key[j] >= thr;
        int total;
        int pos = block_excl_scan(cnt, s_scan, total);
        if (total <= kTopkCandCap) {
#pragma unroll
            for (int j = 0; j < kTopkFastPer; ++j) {
                const int64_t i = (int64_t)j * kTopkThreads + tid;
                if (i < n && key[j] >= thr) s_cand[pos++] = ((uint64_t)key[j] << 32) | (uint32_t)~(uint32_t)i;
            }
            __syncthreads();
            if (total <= 128) {
                // up to 128 candidates: one wave sorts them in registers
                if (wave == 0) {
                    uint64_t k0 = 2 * lane < total ? s_cand[2 * lane] : 0, k1 = 2 * lane + 1 < total ? s_cand[2 * lane + 1] : 0;
                    wave_bitonic128_desc(k0, k1);
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int j = 2 * lane + e;
                        if (j < k) {
                            const int64_t idx = (int64_t)(uint32_t)~(uint32_t)((e ? k1 : k0) & 0xffffffffu);
                            vals[row * k + j] = x[idx];
                            inds[row * k + j] = idx;
                        }
                    }
                }
                return;
            }
            int P = 1;
            while (P < total) P <<= 1;
            for (int i = total + tid; i < P; i += kTopkThreads) s_cand[i] = 0;
            __syncthreads();
            for (int size = 2; size <= P; size <<= 1) {
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    for (int i = tid; i < P / 2; i += kTopkThreads) {
                        const int lo = 2 * i - (i & (stride - 1));
                        const int hi = lo + stride;
                        const bool desc = (lo & size) == 0;
                        const uint64_t a = s_cand[lo], b = s_cand[hi];
                        if ((a < b) == desc) { s_cand[lo] = b; s_cand[hi] = a; }
                    }
                    __syncthreads();
                }
            }
            for (int j = tid; j < k; j += kTopkThreads) {
                const int64_t idx = (int64_t)(uint32_t)~(uint32_t)(s_cand[j] & 0xffffffffu);
                vals[row * k + j] = x[idx];
                inds[row * k + j] = idx;
            }
            return;
        }
        // too many keys tie at the threshold: the general path below
    }

    if (tid == 0) { s_prefix = 0; s_mask = 0; s_remaining = k; }
    __syncthreads();
    // Radix select: after the loop, keys > prefix are strictly selected and
    // `remaining` keys equal to prefix complete the top k.
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int64_t i = tid; i < n; i += kTopkThreads) {
            const uint32_t key = order_key(load_f(x + i), lg);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
        }
        __syncthreads();
        if (wave == 0) {
            // find the digit d (from 255 down) where the running count reaches `remaining`
            const int rem = s_remaining;
            // each lane owns 4 digits, highest digits in lane 0
            int c[4], cs = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) { c[j] = hist[255 - (lane * 4 + j)]; cs += c[j]; }
            int incl = cs;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int y = __shfl_up(incl, off, 64);
                if (lane >= off) incl += y;
            }
            int before = incl - cs;   // count of keys in higher digits than this lane's
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (before < rem && before + c[j] >= rem) {
                    const uint32_t d = 255 - (lane * 4 + j);
                    s_prefix = prefix | (d << shift);
                    s_mask = mask | (255u << shift);
                    s_remaining = rem - before;
                }
                before += c[j];
            }
        }
        __syncthreads();
    }
    const uint32_t thr = s_prefix;
    const int n_eq_take = s_remaining;        // keys == thr to take (lowest indices)
    const int n_gt = k - n_eq_take;

    // Gather the selected (key, index) pairs in index order: thread t owns the
    // contiguous segment [t * per, (t + 1) * per); two block scans of the
    // per-thread counts place them.
    {
        const int64_t per = (n + kTopkThreads - 1) / kTopkThreads;
        const int64_t lo = (int64_t)tid * per, hi = min(n, lo + per);
        int cgt = 0, ceq = 0;
        for (int64_t i = lo; i < hi; ++i) {
            const uint32_t key = order_key(load_f(x + i), lg);
            cgt += key > thr;
            ceq += key == thr;
        }
        // Tie counts only matter below n_eq_take <= 1024: clamping each thread's
        // count to 1024 keeps every prefix exact below 1024 and >= 1024 above.
        int total;
        int pg = block_excl_scan(cgt, s_scan, total);
        int pe = block_excl_scan(min(ceq, kTopkMaxK), s_scan, total);
        for (int64_t i = lo; i < hi; ++i) {
            const uint32_t key = order_key(load_f(x + i), lg);
            const uint64_t comp = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
            if (key > thr) s_sel[pg++] = comp;
            else if (key == thr) {
                if (pe < n_eq_take) s_sel[n_gt + pe] = comp;
                ++pe;
            }
        }
    }
    __syncthreads();

    // Bitonic sort (descending composite) over the next power of two >= k.
    int P = 1;
    while (P < k) P <<= 1;
    for (int i = k + tid; i < P; i += kTopkThreads) s_sel[i] = 0;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < P / 2; i += kTopkThreads) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t a = s_sel[lo], b = s_sel[hi];
                if ((a < b) == desc) { s_sel[lo] = b; s_sel[hi] = a; }
            }
            __syncthreads();
        }
    }
    for (int j = tid; j < k; j += kTopkThreads) {
        const int64_t idx = (int64_t)(uint32_t)~(uint32_t)(s_sel[j] & 0xffffffffu);
        vals[row * k + j] = x[idx];
        inds[row * k + j] = idx;
    }
}

size_t topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
    (void)rows; (void)n; (void)k;
    return 0;
}

// ------------------------------------------------- greedy decode tail

// softmax + top-1 of one row per work-group (rows of at most 32 K
// elements; the arithmetic of softmax_row_kernel's register-cached path, so
// the probabilities are bitwise those of the softmax kernel), then the
// decode-state advance of that row (softmax_top1_row).
template <typename T>
__global__ __launch_bounds__(kSmThreads) void softmax_top1_kernel(int64_t n, const T *X, float *prob, int64_t *index,
                                                                   int32_t *pos, int32_t *kv_len, int64_t *history,
                                                                   int64_t hist_len) {
    const int64_t row = blockIdx.x;
    softmax_top1_row<T, kSmThreads>(n, X + row * n, prob ? prob + row : nullptr, index + row,
                                    pos ? pos + row : nullptr, kv_len ? kv_len + row : nullptr,
                                    history ? history + row * hist_len : nullptr, hist_len);
}

}  // namespace kuiops

using namespace kuiops;

template <typename T>
static void softmax_launch(int64_t m, int64_t n, const void *X, void *Y, hipStream_t st) {
    if (n <= 1024)
        hipLaunchKernelGGL(softmax_wave_kernel<T>, dim3((unsigned)cdiv(m, 4)), dim3(256), 0, st, m, n,
                           (const T *)X, (T *)Y);
    else
        hipLaunchKernelGGL(softmax_row_kernel<T>, dim3((unsigned)m), dim3(kSmThreads), 0, st, n,
                           (const T *)X, (T *)Y);
}

extern "C" int kuiops_softmax_lastdim(int64_t m, int64_t n, int dtype, const void *X, void *Y, void *stream) {
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!X || !Y) return KUIOPS_E_INVALID;
    if (m > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case KUIOPS_F32: softmax_launch<float>(m, n, X, Y, st); break;
        case KUIOPS_BF16: softmax_launch<bf16_t>(m, n, X, Y, st); break;
        case KUIOPS_F16: softmax_launch<f16_t>(m, n, X, Y, st); break;
        case KUIOPS_F64: softmax_launch<double>(m, n, X, Y, st); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

extern "C" int kuiops_topk_lastdim(int64_t m, int64_t n, int64_t k, int dtype, const void *X, void *values,
                                   int64_t *indices, int largest, int sorted, void *workspace,
                                   size_t workspace_bytes, void *stream) {
    (void)sorted; (void)workspace; (void)workspace_bytes;
    if (m < 0 || n < 0 || k < 0 || k > n) return KUIOPS_E_INVALID;
    if (m == 0 || k == 0) return KUIOPS_OK;
    if (!X || !values || !indices) return KUIOPS_E_INVALID;
    if (k > kTopkMaxK || n >= (int64_t)UINT32_MAX || m > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    dim3 grid((unsigned)m), block(kTopkThreads);
    switch (dtype) {
        case KUIOPS_F32: hipLaunchKernelGGL(topk_kernel<float>, grid, block, 0, st, n, (int)k, (const float *)X, (float *)values, indices, largest); break;
        case KUIOPS_BF16: hipLaunchKernelGGL(topk_kernel<bf16_t>, grid, block, 0, st, n, (int)k, (const bf16_t *)X, (bf16_t *)values, indices, largest); break;
        case KUIOPS_F16: hipLaunchKernelGGL(topk_kernel<f16_t>, grid, block, 0, st, n, (int)k, (const f16_t *)X, (f16_t *)values, indices, largest); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

extern "C" int kuiops_softmax_top1(int64_t m, int64_t n, int dtype, const void *X, float *prob, int64_t *index,
                                   int32_t *pos, int32_t *kv_len, int64_t *history, int64_t hist_len, void *stream) {
    if (history && (hist_len <= 0 || !pos)) return KUIOPS_E_INVALID;
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0) return KUIOPS_OK;
    if (n == 0 || !X || !index) return KUIOPS_E_INVALID;
    if (n > (int64_t)kSmThreads * kSmCache || m > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)m);
    switch (dtype) {
        case KUIOPS_F32: hipLaunchKernelGGL(softmax_top1_kernel<float>, grid, dim3(kSmThreads), 0, st, n, (const float *)X, prob, index, pos, kv_len, history, hist_len); break;
        case KUIOPS_BF16: hipLaunchKernelGGL(softmax_top1_kernel<bf16_t>, grid, dim3(kSmThreads), 0, st, n, (const bf16_t *)X, prob, index, pos, kv_len, history, hist_len); break;
        case KUIOPS_F16: hipLaunchKernelGGL(softmax_top1_kernel<f16_t>, grid, dim3(kSmThreads), 0, st, n, (const f16_t *)X, prob, index, pos, kv_len, history, hist_len); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}
