// One greedy decode step of a Llama-style decoder (batch 1) in a single
// persistent launch.
//
// The per-op decode step is ~5 launches per layer (qkv + rotary + KV append,
// attention, o, gate|up + SwiGLU, down) plus the LM head and the sampling
// tail: ~82 dependent launches per token for a 16-layer model, each paying a
// few microseconds of launch, ramp-up and drain on top of its weight
// streaming.  Here one launch of one 8-wave work-group per CU walks the same
// work as an ordered list of jobs:
//
//   per layer   qkv row blocks | attention rows (one per query head) |
//               o row blocks | gate|up row blocks | down row blocks
//   then        LM-head row blocks | the softmax + top-1 row
//
// Work-group w takes jobs w, w + G, w + 2G, ... (G = grid size).  A job of
// phase p needs every job of phase p - 1 (the next projection's input is the
// whole previous vector: RMSNorm needs the full row); it issues its weight
// loads first, then waits on the phase's completion counters, so the weight
// stream of later phases runs while earlier phases finish.  Jobs only wait on
// jobs with lower indices, so with all G work-groups resident (one per CU,
// nothing else running) the lowest unfinished job can always run: the step
// cannot deadlock.  Every wait is bounded; on expiry the step stops waiting,
// sets the error word and runs to the end (results undefined, no hang).
//
// Ordering: every activation a job hands to another job (projection
// outputs, the new K / V rows, attention rows, logits) is written with
// agent-scope relaxed atomic stores (sc1: written through the per-XCD L2)
// and read with agent-scope relaxed atomic loads (sc1: served past the
// non-coherent caches).  A finished job's threads wait for their stores'
// acknowledgements (s_waitcnt 0) before the work-group barrier that
// precedes one relaxed agent-scope add on a completion counter; a waiting
// work-group polls the counters with relaxed agent-scope loads and its
// barrier precedes its input reads.  This relies on the gfx942 / gfx950
// rule that an acknowledged sc1 store is visible at the agent's coherence
// point before a later atomic of the same agent (the rule the split-K
// merges of the decode GEMM and decode attention use); release / acquire
// fences would write back / invalidate the whole L2 per job, which costs
// more than the step itself (measured 2.5 ms against 0.9 ms per token).
// Weights and the older cache rows are read with ordinary loads: nothing
// in the launch writes them.

// The job bodies are the library's own (decode_rows_block, fa_decode_block,
// softmax_top1_row), with the launch shapes and summation orders of the
// per-op kernels, so the step is bitwise the per-op sequence.
#include "attn_decode.hpp"
#include "top1.hpp"
#include "decode_rows.hpp"

namespace kuiops {

constexpr int kStepWaves = 8;
constexpr int kStepThreads = kStepWaves * 64;
constexpr int kKinds = 7;                 // qkv, attention, o, gate|up, down, LM head, sampling
constexpr int kLayerKinds = 5;
constexpr int kSubCounters = 8;           // completion counters per phase (spread contention)
constexpr int kCounterStride = 32;        // uint32 apart: one 128-byte line each
constexpr unsigned kSpinLimit = 1u << 20; // polls per wait (~1 s)

struct StepArgs {
    int layers;
    int64_t d, ffn, hq, hkv, hd, vocab, cap;
    int64_t sk1, sk2, sv1, sv2;
    float eps, scale_log2;
    int shift_hd, shift_ffn;              // log2(hd / 2), log2(ffn) or -1
    const kuiops_step_layer *layer;
    const void *embed, *norm, *head;
    const float *inv_freq;
    int64_t *tok;
    int32_t *pos, *kv_len;
    int64_t *history;
    int64_t hist_len;
    float *prob;
    void *h0, *h1, *q, *att, *o, *act, *down, *logits;
    unsigned *sync;
    int njobs[kKinds];
    int per_layer, total;
};

__device__ __forceinline__ int n_phases(const StepArgs &a) { return kLayerKinds * a.layers + 2; }

__device__ __forceinline__ unsigned *counter_of(const StepArgs &a, int phase, int k) {
    return a.sync + ((int64_t)phase * kSubCounters + k) * kCounterStride;
}
__device__ __forceinline__ unsigned *error_word(const StepArgs &a) {
    return a.sync + (int64_t)n_phases(a) * kSubCounters * kCounterStride;
}

__device__ __forceinline__ int kind_of_phase(const StepArgs &a, int phase) {
    const int lp = kLayerKinds * a.layers;
    return phase < lp ? phase % kLayerKinds : kLayerKinds + (phase - lp);
}

// Waits until every job of `phase` has signalled (phase < 0: nothing to wait
// for).  Wave 0 polls the phase's counters (lanes 0..7) and the error word
// (lane 8); all threads leave through the barrier.
__device__ __forceinline__ void step_wait(const StepArgs &a, int phase) {
    if (phase < 0) return;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const unsigned need = (unsigned)a.njobs[kind_of_phase(a, phase)];
        for (unsigned it = 0;; ++it) {
            unsigned v = 0, err = 0;
            if (lane < kSubCounters)
                v = __hip_atomic_load(counter_of(a, phase, lane), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else if (lane == kSubCounters)
                err = __hip_atomic_load(error_word(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v += __shfl_xor(v, 1, 64);
            v += __shfl_xor(v, 2, 64);
            v += __shfl_xor(v, 4, 64);
            v = __shfl(v, 0, 64);
            err = __shfl(err, kSubCounters, 64);
            if (v >= need || err) break;
            if (it >= kSpinLimit) {
                if (lane == 0) __hip_atomic_store(error_word(a), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

// Publishes the calling work-group's job `idx` of `phase`.
__device__ __forceinline__ void step_signal(const StepArgs &a, int phase, int idx) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(counter_of(a, phase, idx % kSubCounters), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

struct StepWait {
    const StepArgs *a;
    int phase;
    __device__ __forceinline__ void operator()() const { step_wait(*a, phase); }
};

// Rows per wave of a projection job: 32 registers of W chunks (128 VGPRs),
// so a work-group holds 128-256 KB of weights in flight while it waits; the
// large projections (gate|up, down, LM head) hold 16 more chunks per wave in
// LDS (kLdsRowBytes per work-group).  With them the layer's qkv, attention,
// o and gate|up jobs fit one round of the grid, and the down jobs land on
// work-groups that finished early, whose weight loads then run during the
// gate|up phase.
constexpr int rows_per_wave(int kc) { return kc <= 4 ? 8 : (kc <= 8 ? 4 : 2); }
constexpr int lds_rows_per_wave(int kc) { return kc <= 4 ? 4 : (kc <= 8 ? 2 : 1); }
constexpr int kLdsRowBytes = kStepWaves * 16 * 1024;
constexpr int kLdsXBytes = kDecodeMaxK * 2;         // the staged input x

// The projection of layer `l` of one kind, as the per-op entry points set it up.
__device__ __forceinline__ DecLinArgs proj_args(const StepArgs &a, int kind, int l, int rpw) {
    DecLinArgs p{};
    p.eps = a.eps;
    p.rpw = rpw;
    p.pair_shift = -1;
    if (kind == 5) {                      // LM head: RMSNorm(h0 + down) input
        p.N = a.vocab; p.K = a.d;
        p.in = a.h0; p.in_add = a.down; p.norm_w = a.norm;
        p.W = a.head; p.ldw = a.d; p.out = a.logits;
        return p;
    }
    const kuiops_step_layer &L = a.layer[l];
    switch (kind) {
        case 0:                           // qkv: RMSNorm(h0 + down) (layer 0: the embedding row), rotary + KV
            p.N = (a.hq + 2 * a.hkv) * a.hd; p.K = a.d;
            if (l == 0) {
                p.in = a.embed; p.in_row = a.tok; p.ld_in = a.d; p.in_rows = a.vocab;
            } else {
                p.in = a.h0; p.in_add = a.down;
            }
            p.norm_w = L.ln1; p.h_out = a.h1;
            p.W = L.wqkv; p.ldw = a.d; p.out = a.q;
            p.pair_off = a.hd / 2; p.pair_shift = a.shift_hd;
            p.hq = a.hq; p.hkv = a.hkv; p.hd = a.hd; p.inv_freq = a.inv_freq; p.pos = a.pos;
            p.kc = L.k_cache; p.sk1 = a.sk1; p.sk2 = a.sk2;
            p.vc = L.v_cache; p.sv1 = a.sv1; p.sv2 = a.sv2;
            p.cap = a.cap;
            break;
        case 2:                           // o: plain input (the attention rows)
            p.N = a.d; p.K = a.hq * a.hd;
            p.in = a.att; p.W = L.wo; p.ldw = a.hq * a.hd; p.out = a.o;
            break;
        case 3:                           // gate|up: RMSNorm(h1 + o), SwiGLU pairs
            p.N = 2 * a.ffn; p.K = a.d;
            p.in = a.h1; p.in_add = a.o; p.norm_w = L.ln2; p.h_out = a.h0;
            p.W = L.wgu; p.ldw = a.d; p.out = a.act;
            p.pair_off = a.ffn; p.pair_shift = a.shift_ffn;
            break;
        default:                          // down: plain input (the SwiGLU activations)
            p.N = a.d; p.K = a.ffn;
            p.in = a.act; p.W = L.wd; p.ldw = a.ffn; p.out = a.down;
            break;
    }
    return p;
}

// The job kinds, each its own function: inlined into one loop, the bodies'
// register demands add up (spills); as calls each gets its own allocation.
template <typename T, int XK, int KC, int OK, int RGL = 0>
__device__ __attribute__((noinline)) void step_proj(const StepArgs &a, int kind, int l, int idx, int phase,
                                                    lds_bytes *wl) {
    decode_rows_block<T, XK, KC, OK, kStepWaves, StepWait, CoherentIO, rows_per_wave(KC), RGL, true>(
        proj_args(a, kind, l, rows_per_wave(KC) + RGL), idx, StepWait{&a, phase - 1}, wl, wl + kLdsRowBytes);
}

// attention row `idx` (query head) of layer l, as the per-op row-wide launch
// runs it: one work-group per query row, every key in one pass.  The cache
// rows before this token's position do not depend on the qkv phase: their
// loads are issued before the wait, and the row at the position (written by
// the qkv phase) is read again after it.
template <typename T, int HD>
__device__ __attribute__((noinline)) void step_attention(const StepArgs &a, int l, int idx, int phase) {
    const int64_t fresh = *a.pos;
    const kuiops_step_layer &L = a.layer[l];
    AttnArgs at{};
    at.n = 1; at.hq = a.hq; at.hkv = a.hkv; at.l = 1; at.s = a.cap;
    at.Q = a.q; at.K = L.k_cache; at.V = L.v_cache; at.O = a.att;
    at.sq0 = a.hq * a.hd; at.sq1 = a.hd; at.sq2 = a.hd;
    at.sk0 = 0; at.sk1 = a.sk1; at.sk2 = a.sk2;
    at.sv0 = 0; at.sv1 = a.sv1; at.sv2 = a.sv2;
    at.so0 = a.hq * a.hd; at.so1 = a.hd; at.so2 = a.hq * a.hd;
    at.scale_log2 = a.scale_log2;
    at.causal = 1;
    at.splits = 1; at.chunk = a.cap;
    at.rows_per_group = 1; at.row_groups = (int)(a.hq / a.hkv);
    at.kv_len = a.kv_len;
    fa_decode_block<T, HD, 1, kStepWaves, 12, CoherentIO, StepWait, true>(at, 0, idx, 0, StepWait{&a, phase - 1}, fresh);
}

// softmax + top-1 of the logits and the decode-state advance; every other
// job has finished by then (each phase waited on the one before it), so the
// counters are left zero for the next step
template <typename T>
__device__ __attribute__((noinline)) void step_sample(const StepArgs &a, int phase) {
    step_wait(a, phase - 1);
    softmax_top1_row<T, kStepThreads, CoherentIO>(a.vocab, reinterpret_cast<const T *>(a.logits), a.prob, a.tok, a.pos,
                                      a.kv_len, a.history, a.hist_len);
    __syncthreads();
    for (int i = threadIdx.x; i < n_phases(a) * kSubCounters; i += kStepThreads)
        __hip_atomic_store(a.sync + (int64_t)i * kCounterStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int HD, int KCD, int KCF>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepArgs a) {
    constexpr int RLD = lds_rows_per_wave(KCD), RLF = lds_rows_per_wave(KCF);
    __shared__ __attribute__((aligned(1024))) char s_wl[kLdsRowBytes + kLdsXBytes];
    lds_bytes *wl = (lds_bytes *)s_wl;
    const int G = gridDim.x;
    const int lp = kLayerKinds * a.layers;
    for (int j = blockIdx.x; j < a.total; j += G) {
        int l, kind, idx, phase;
        if (j < a.layers * a.per_layer) {
            l = j / a.per_layer;
            idx = j - l * a.per_layer;
            kind = 0;
            while (idx >= a.njobs[kind]) idx -= a.njobs[kind++];
            phase = l * kLayerKinds + kind;
        } else {
            l = a.layers;
            idx = j - a.layers * a.per_layer;
            kind = idx < a.njobs[5] ? 5 : 6;
            if (kind == 6) idx -= a.njobs[5];
            phase = lp + (kind - kLayerKinds);
        }
        switch (kind) {
            case 0: step_proj<T, kXRmsNorm, KCD, kOutRope>(a, 0, l, idx, phase, wl); break;
            case 1: step_attention<T, HD>(a, l, idx, phase); break;
            case 2: step_proj<T, kXPlain, KCD, kOutPlain>(a, 2, l, idx, phase, wl); break;
            case 3: step_proj<T, kXRmsNorm, KCD, kOutSwiGlu, RLD>(a, 3, l, idx, phase, wl); break;
            case 4: step_proj<T, kXPlain, KCF, kOutPlain, RLF>(a, 4, l, idx, phase, wl); break;
            case 5: step_proj<T, kXRmsNorm, KCD, kOutPlain, RLD>(a, 5, l, idx, phase, wl); break;
            default: step_sample<T>(a, phase); continue;
        }
        step_signal(a, phase, idx);
    }
}

static int kc_bucket(int64_t K) {
    const int64_t kc = cdiv(K, 512);
    return kc <= 4 ? 4 : kc <= 8 ? 8 : kc <= 12 ? 12 : kc <= 16 ? 16 : 0;
}

static int log2_of(int64_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int k = 0;
    while ((int64_t(1) << k) < v) ++k;
    return k;
}

template <typename T, int HD, int KCD>
static void launch_step_kcf(const StepArgs &a, int kcf, dim3 grid, hipStream_t st) {
    switch (kcf) {
        case 4: hipLaunchKernelGGL((decode_step_kernel<T, HD, KCD, 4>), grid, dim3(kStepThreads), 0, st, a); break;
        case 8: hipLaunchKernelGGL((decode_step_kernel<T, HD, KCD, 8>), grid, dim3(kStepThreads), 0, st, a); break;
        case 12: hipLaunchKernelGGL((decode_step_kernel<T, HD, KCD, 12>), grid, dim3(kStepThreads), 0, st, a); break;
        default: hipLaunchKernelGGL((decode_step_kernel<T, HD, KCD, 16>), grid, dim3(kStepThreads), 0, st, a); break;
    }
}

template <typename T>
static void launch_step(const StepArgs &a, int kcd, int kcf, dim3 grid, hipStream_t st) {
    if (a.hd == 64) {
        if (kcd == 4) launch_step_kcf<T, 64, 4>(a, kcf, grid, st);
        else launch_step_kcf<T, 64, 8>(a, kcf, grid, st);
    } else {
        if (kcd == 4) launch_step_kcf<T, 128, 4>(a, kcf, grid, st);
        else launch_step_kcf<T, 128, 8>(a, kcf, grid, st);
    }
}

}  // namespace kuiops

using namespace kuiops;

extern "C" size_t kuiops_decode_step_sync_bytes(int64_t n_layers) {
    if (n_layers < 0) return 0;
    return (size_t)((kLayerKinds * n_layers + 2) * kSubCounters + 1) * kCounterStride * sizeof(unsigned);
}

extern "C" int kuiops_decode_step(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv, int64_t hd,
                                  int64_t vocab, int64_t cache_cap, int dtype, float eps,
                                  const kuiops_step_layer *layers, int64_t sk_head, int64_t sk_pos,
                                  int64_t sv_head, int64_t sv_pos, const void *embed, const void *final_norm,
                                  const void *lm_head, const float *inv_freq, int64_t *tok, int32_t *pos,
                                  int32_t *kv_len, int64_t *history, int64_t hist_len, float *prob, void *h0,
                                  void *h1, void *q, void *att, void *o, void *act, void *down, void *logits,
                                  void *sync, size_t sync_bytes, void *stream) {
    if (n_layers <= 0 || d <= 0 || ffn <= 0 || hq <= 0 || hkv <= 0 || hd <= 0 || vocab <= 0 || cache_cap <= 0)
        return KUIOPS_E_INVALID;
    if (hq % hkv || hd % 2) return KUIOPS_E_INVALID;
    if (!layers || !embed || !final_norm || !lm_head || !inv_freq || !tok || !pos || !kv_len || !h0 || !h1 ||
        !q || !att || !o || !act || !down || !logits || !sync)
        return KUIOPS_E_INVALID;
    if (history && hist_len <= 0) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if ((hd != 64 && hd != 128) || d != hq * hd || d % 8 || ffn % 8) return KUIOPS_E_UNSUPPORTED;
    const int kcd = kc_bucket(d), kcf = kc_bucket(ffn);
    if (kcd == 0 || kcd > 8 || kcf == 0) return KUIOPS_E_UNSUPPORTED;   // paired epilogues: d <= 4096
    if (vocab > (int64_t)kSmThreads * kSmCache || vocab > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    if (n_layers > 1024 || cache_cap > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    if (sync_bytes < kuiops_decode_step_sync_bytes(n_layers) || !aligned16(sync)) return KUIOPS_E_WORKSPACE;
    for (const void *p : {embed, final_norm, lm_head, (const void *)h0, (const void *)h1, (const void *)q,
                          (const void *)att, (const void *)o, (const void *)act, (const void *)down,
                          (const void *)logits})
        if (!aligned16(p)) return KUIOPS_E_UNSUPPORTED;
    if (sk_pos % 8 || sv_pos % 8 || sk_head % 8 || sv_head % 8) return KUIOPS_E_UNSUPPORTED;

    StepArgs a{};
    a.layers = (int)n_layers;
    a.d = d; a.ffn = ffn; a.hq = hq; a.hkv = hkv; a.hd = hd; a.vocab = vocab; a.cap = cache_cap;
    a.sk1 = sk_head; a.sk2 = sk_pos; a.sv1 = sv_head; a.sv2 = sv_pos;
    a.eps = eps;
    // the softmax scale 1/sqrt(hd) as the per-op attention receives it (fp32)
    const float scale = (float)(1.0 / __builtin_sqrt((double)hd));
    a.scale_log2 = scale * 1.44269504088896340736f;
    a.shift_hd = log2_of(hd / 2);
    a.shift_ffn = log2_of(ffn);
    a.layer = layers;
    a.embed = embed; a.norm = final_norm; a.head = lm_head; a.inv_freq = inv_freq;
    a.tok = tok; a.pos = pos; a.kv_len = kv_len; a.history = history; a.hist_len = hist_len; a.prob = prob;
    a.h0 = h0; a.h1 = h1; a.q = q; a.att = att; a.o = o; a.act = act; a.down = down; a.logits = logits;
    a.sync = reinterpret_cast<unsigned *>(sync);
    const int64_t rows_d = (int64_t)kStepWaves * rows_per_wave(kcd);
    const int64_t rows_dl = (int64_t)kStepWaves * (rows_per_wave(kcd) + lds_rows_per_wave(kcd));
    const int64_t rows_fl = (int64_t)kStepWaves * (rows_per_wave(kcf) + lds_rows_per_wave(kcf));
    const int64_t nj[kKinds] = {cdiv((hq + 2 * hkv) * hd, rows_d), hq, cdiv(d, rows_d), cdiv(2 * ffn, rows_dl),
                                cdiv(d, rows_fl), cdiv(vocab, rows_dl), 1};
    int64_t per_layer = 0;
    for (int k = 0; k < kLayerKinds; ++k) per_layer += nj[k];
    const int64_t total = n_layers * per_layer + nj[5] + nj[6];
    if (total > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    for (int k = 0; k < kKinds; ++k) a.njobs[k] = (int)nj[k];
    a.per_layer = (int)per_layer;
    a.total = (int)total;
    // one work-group per CU: all resident at once (a job waits only on jobs
    // with lower indices, which resident work-groups run)
    const dim3 grid((unsigned)num_cus());
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) launch_step<bf16_t>(a, kcd, kcf, grid, st);
    else launch_step<f16_t>(a, kcd, kcf, grid, st);
    return launch_status();
}

extern "C" int kuiops_decode_step_error(void *sync, int64_t n_layers, void *stream) {
    if (!sync || n_layers <= 0) return KUIOPS_E_INVALID;
    unsigned *w = reinterpret_cast<unsigned *>(sync) + (kLayerKinds * n_layers + 2) * kSubCounters * kCounterStride;
    unsigned v = 0;
    hipStream_t st = as_stream(stream);
    if (hipMemcpyAsync(&v, w, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess) return KUIOPS_E_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return KUIOPS_E_HIP;
    if (v && hipMemsetAsync(w, 0, sizeof(unsigned), st) != hipSuccess) return KUIOPS_E_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return KUIOPS_E_HIP;
    return v ? 1 : 0;
}
