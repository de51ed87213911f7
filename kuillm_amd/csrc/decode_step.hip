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
//   then        LM-head row blocks (one full-size block per work-group,
//               the rest in small blocks) | the softmax + top-1 row
//
// Work-group w takes jobs w, w + G, w + 2G, ... (G = grid size).  A job of
// phase p needs the whole output of phase p - 1 (the next projection's input
// is the whole previous vector: RMSNorm needs the full row); it issues its
// weight loads first (and attention its older cache rows), then waits for its
// input, so the weight stream of later phases runs while earlier phases
// finish.  Jobs only wait on jobs with lower indices, so with all G
// work-groups resident (one per CU, nothing else running) the lowest
// unfinished job can always run: the step cannot deadlock.  Every wait is
// bounded; on expiry the step stops waiting, sets the error word and runs to
// the end (results undefined, no hang).  The error word latches: a launch
// that finds it set does no work, until the host reads and clears it
// (kuiops_decode_step_error).  Before launching, the host refuses shapes
// whose work-group does not fit a CU (occupancy query) and caches longer
// than the one-pass attention covers.
//
// Hand-off: the vectors that pass between jobs (residual, q, attention rows,
// o, SwiGLU activations, down, the new k / v rows, the sampled token) are
// epoch-tagged: each 8-byte word holds two elements and the epoch of its
// write (step counter x layer), written with agent-coherent stores (sc1:
// through the per-XCD L2; 8 elements as two 16-byte stores, each 8-byte word
// whole).  A consumer's waves read their chunks, probe the first word of a
// chunk that is not yet the expected write and read it again, until every
// word carries the epoch they expect; then the work-group meets at a
// barrier.  So a hand-off costs no store acknowledgement wait, no counter
// and no separate poll: the reader detects the data itself.  Only the LM
// head's logits (read by the sampling job) go through completion counters
// (stores acknowledged with s_waitcnt 0, barrier, one relaxed agent-scope
// add; the rule the split-K merges use).  The KV cache rows are written with
// ordinary stores (read by later launches; this launch's attention takes the
// rows of this launch's steps from their epoch-tagged copies), and weights
// and older cache rows are read with ordinary loads: nothing in the launch
// writes them.
//
// A launch can run several steps: the job list repeats per step, the
// position and key count of step t are the launch's starting values plus t,
// and the sampled token reaches the next step's layer-0 jobs as an
// epoch-tagged word.
//
// The job bodies are the library's own (decode_rows_block, fa_decode_onepass_block,
// softmax_top1_row), with the launch shapes and summation orders of the
// per-op kernels, so the step is bitwise the per-op sequence.
#include <algorithm>

#include "attn_decode.hpp"
#include "top1.hpp"
#include "decode_rows.hpp"

namespace kuiops {

constexpr int kStepWaves = 8;
constexpr int kStepThreads = kStepWaves * 64;
constexpr int kKinds = 8;                 // qkv, attention, o, gate|up, down, LM head (two sizes), sampling
constexpr int kHeadTailRows = 4;          // rows per wave of the LM head's second-round jobs
constexpr int kLayerKinds = 5;
constexpr int kSubCounters = 8;           // completion counters of the LM-head phase (spread contention)
constexpr int kCounterStride = 32;        // uint32 apart: one 128-byte line each
constexpr unsigned kSpinLimit = 1u << 20; // polls per wait (~1 s)
constexpr int kMaxSteps = 32;             // tokens per launch (the window of fresh keys, at most 31,
                                           // is narrower than the 32-key spacing of a lane's keys)

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
    void *h0, *h1, *q, *att, *o, *act, *down;   // epoch-tagged (scratch)
    void *kf, *vf;                        // epoch-tagged new k / v rows, [layers][steps][hkv * hd]
    void *logits;
    unsigned *sync;
    int njobs[kKinds];
    int per_layer, per_token, steps, total;
    int64_t head_split;                   // LM-head rows of the full-size jobs (kind 5); kind 6 takes the rest
};

// The job functions take the launch's arguments by reference.  (The
// compiler gives the kernel's by-value parameter a per-lane copy in scratch
// for it; measured against a constant- or LDS-address-space reference,
// whose bodies spill, this is the faster form.)
typedef const StepArgs &StepArgsRef;

// sync: kSubCounters counters of the LM-head phase, the error word, the step
// epoch, the epoch-tagged sampled token (one 128-byte line each)
__device__ __forceinline__ unsigned *counter_of(StepArgsRef a, int k) { return a.sync + k * kCounterStride; }
__device__ __forceinline__ unsigned *error_word(StepArgsRef a) { return a.sync + kSubCounters * kCounterStride; }
__device__ __forceinline__ unsigned *epoch_word(StepArgsRef a) { return a.sync + (kSubCounters + 1) * kCounterStride; }
__device__ __forceinline__ void *token_word(StepArgsRef a) { return a.sync + (kSubCounters + 2) * kCounterStride; }

// Token t of a launch: its step (epoch counter), position and key count.
// Each sampling job advances the position and the key count by one, so
// token t's are the launch's starting values plus t.
struct StepTok {
    int t;
    uint32_t step;
    int64_t pos, kv;
};

// The epoch-tagged new k / v rows of layer l, token t (element offset).
__device__ __forceinline__ int64_t fresh_slot(StepArgsRef a, int l, int t) {
    return ((int64_t)l * a.steps + t) * a.hkv * a.hd;
}

// Epoch of the vectors written by layer l (l = layers: none) in this step.
__device__ __forceinline__ uint32_t epoch_of(StepArgsRef a, uint32_t step, int l) {
    return step * (uint32_t)(a.layers + 1) + (uint32_t)l + 1u;
}

// Waits until every LM-head job of tokens 0 .. t has signalled (the
// counters accumulate over the launch).  Wave 0 polls the counters (lanes
// 0..7) and the error word (lane 8); all threads leave through the barrier.
__device__ __forceinline__ void wait_head(StepArgsRef a, int t) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const unsigned need = (unsigned)((t + 1) * (a.njobs[5] + a.njobs[6]));
        for (unsigned it = 0;; ++it) {
            unsigned v = 0, err = 0;
            if (lane < kSubCounters)
                v = __hip_atomic_load(counter_of(a, lane), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Publishes the calling work-group's LM-head job `idx`.
__device__ __forceinline__ void signal_head(StepArgsRef a, int idx) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(counter_of(a, idx % kSubCounters), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


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
__device__ __forceinline__ DecLinArgs proj_args(StepArgsRef a, int kind, int l, int rpw, const StepTok tk) {
    const uint32_t step = tk.step;
    DecLinArgs p{};
    p.eps = a.eps;
    p.rpw = rpw;
    p.pair_shift = -1;
    p.err = error_word(a);
    if (kind >= 5) {                      // LM head: RMSNorm(h0 + down) input; kind 6 from row head_split
        const int64_t r0 = kind == 6 ? a.head_split : 0;
        p.N = a.vocab - r0; p.K = a.d;
        p.in = a.h0; p.in_add = a.down; p.norm_w = a.norm;
        p.ep_in = p.ep_add = epoch_of(a, step, a.layers - 1);
        p.W = reinterpret_cast<const char *>(a.head) + r0 * a.d * 2; p.ldw = a.d;
        p.out = reinterpret_cast<char *>(a.logits) + r0 * 2;
        return p;
    }
    // inputs from this layer's earlier phases, or (qkv) the previous layer's
    p.ep_in = p.ep_add = epoch_of(a, step, kind == 0 ? l - 1 : l);
    p.ep_out = epoch_of(a, step, l);
    const kuiops_step_layer &L = a.layer[l];
    switch (kind) {
        case 0:                           // qkv: RMSNorm(h0 + down) (layer 0: the embedding row), rotary + KV
            p.N = (a.hq + 2 * a.hkv) * a.hd; p.K = a.d;
            if (l == 0) {
                // the embedding row of the token: from the previous launch, or
                // (later tokens) from this launch's sampling job
                p.in = a.embed; p.ld_in = a.d; p.in_rows = a.vocab;
                if (tk.t == 0) {
                    p.in_row = a.tok;
                } else {
                    p.row_ll = token_word(a);
                    p.ep_row = step;
                }
            } else {
                p.in = a.h0; p.in_add = a.down;
            }
            p.norm_w = L.ln1; p.h_out = a.h1;
            p.W = L.wqkv; p.ldw = a.d; p.out = a.q;
            p.pair_off = a.hd / 2; p.pair_shift = a.shift_hd;
            p.hq = a.hq; p.hkv = a.hkv; p.hd = a.hd; p.inv_freq = a.inv_freq;
            p.use_pos_val = 1; p.pos_val = tk.pos;
            p.kc = L.k_cache; p.sk1 = a.sk1; p.sk2 = a.sk2;
            p.vc = L.v_cache; p.sv1 = a.sv1; p.sv2 = a.sv2;
            p.cap = a.cap;
            p.kfresh = reinterpret_cast<char *>(a.kf) + fresh_slot(a, l, tk.t) * 4;   // (2 elements per 8 bytes)
            p.vfresh = reinterpret_cast<char *>(a.vf) + fresh_slot(a, l, tk.t) * 4;
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
template <typename T, int XK, int KC, int OK, int RGL, typename IO, typename OIO, int RG = rows_per_wave(KC)>
__device__ __attribute__((noinline)) void step_proj(StepArgsRef a, int kind, int l, int idx, const StepTok tk,
                                                    lds_bytes *wl) {
    decode_rows_block<T, XK, KC, OK, kStepWaves, NoWait, IO, RG, RGL, true, OIO>(
        proj_args(a, kind, l, RG + RGL, tk), idx, NoWait{}, wl, wl + kLdsRowBytes);
}

// attention row `idx` (query head) of layer l, as the per-op row-wide launch
// runs it: one work-group per query row, every key in one pass.  The cache
// rows written by earlier launches do not depend on the qkv phase: their
// loads are issued before the query is awaited; the rows of this launch's
// tokens (positions pos - t .. pos) come from the qkv phases' epoch-tagged
// copies.
template <typename T, int HD>
__device__ __attribute__((noinline)) void step_attention(StepArgsRef a, int l, int idx, const StepTok tk) {
    // (the qkv phase writes the new row only when it is inside the cache)
    const int64_t fresh = tk.pos >= 0 && tk.pos < a.cap ? tk.pos : -1;
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
    at.use_s_len = 1; at.s_len = tk.kv;
    at.ep_q = at.ep_o = epoch_of(a, tk.step, l);
    at.kfresh = reinterpret_cast<const char *>(a.kf) + fresh_slot(a, l, 0) * 4;
    at.vfresh = reinterpret_cast<const char *>(a.vf) + fresh_slot(a, l, 0) * 4;
    at.fresh_lo = tk.pos - tk.t; at.fresh_stride = a.hkv * a.hd;
    at.ep_fresh0 = epoch_of(a, tk.step - (uint32_t)tk.t, l); at.ep_fresh_step = (uint32_t)(a.layers + 1);
    at.err = error_word(a);
    fa_decode_onepass_block<T, HD, kStepWaves, 12, LLIO, true>(at, idx, 0, fresh);
}

// softmax + top-1 of token t's logits.  The token goes to history[pos] and,
// for the next token of the launch, to the epoch-tagged token word.  The
// last token's sampling job runs after every other job of the launch has
// finished (each phase waited on the one before it): it writes the decode
// state for the next launch (token, position, key count, probability), zeroes
// the counters and advances the step epoch.
template <typename T>
__device__ __attribute__((noinline)) void step_sample(StepArgsRef a, const StepTok tk, lds_bytes *wl) {
    const bool last = tk.t == a.steps - 1;
    wait_head(a, tk.t);
    __shared__ int64_t s_tok;
    softmax_top1_row<T, kStepThreads, CoherentIO>(a.vocab, reinterpret_cast<const T *>(a.logits),
                                                  last ? a.prob : nullptr, &s_tok, nullptr, nullptr, nullptr, 0, wl);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int64_t i = s_tok;
        if (a.history && tk.pos >= 0 && tk.pos < a.hist_len) a.history[tk.pos] = i;
        if (!last) {
            LLIO::put(token_word(a), 0, (uint32_t)i, tk.step + 1u);
        } else {
            *a.tok = i;
            *a.pos = (int32_t)(tk.pos + 1);
            *a.kv_len = (int32_t)(tk.kv + 1);
            *epoch_word(a) = tk.step + 1u;
        }
    }
    if (last && threadIdx.x < kSubCounters)
        __hip_atomic_store(counter_of(a, threadIdx.x), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Job j of the step's list: layer, kind and index within the kind.
__device__ __forceinline__ void job_of(StepArgsRef a, int j, int &l, int &kind, int &idx) {
    if (j < a.layers * a.per_layer) {
        l = j / a.per_layer;
        idx = j - l * a.per_layer;
        kind = 0;
        while (idx >= a.njobs[kind]) idx -= a.njobs[kind++];
    } else {
        l = a.layers;
        idx = j - a.layers * a.per_layer;
        kind = 5;
        while (kind < kKinds - 1 && idx >= a.njobs[kind]) idx -= a.njobs[kind++];
    }
}

template <typename T, int HD, int KCD, int KCF>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepArgs a) {
    constexpr int RLD = lds_rows_per_wave(KCD), RLF = lds_rows_per_wave(KCF);
    __shared__ __attribute__((aligned(1024))) char s_wl[kLdsRowBytes + kLdsXBytes];
    lds_bytes *wl = (lds_bytes *)s_wl;
    StepArgsRef args = a;
    const int G = gridDim.x;
    // The step counter and the decode state as the previous launch left
    // them: written only by this launch's last sampling job, which runs after
    // every other job has finished (and so every work-group has read them).
    // A latched error (a bounded wait of an earlier launch expired, and the
    // host has not cleared it) voids the decode state: do no work.
    __shared__ unsigned s_err;
    if (threadIdx.x == 0) s_err = __hip_atomic_load(error_word(args), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_err) return;
    const uint32_t step0 = *epoch_word(args);
    const int64_t pos0 = *args.pos, kv0 = *args.kv_len;
    for (int j = blockIdx.x; j < args.total; j += G) {
        const int t = j / args.per_token;
        const StepTok tk{t, step0 + (uint32_t)t, pos0 + t, kv0 + t};
        int l, kind, idx;
        job_of(args, j - t * args.per_token, l, kind, idx);
        switch (kind) {
            case 0:
                if (l == 0) step_proj<T, kXRmsNorm, KCD, kOutRope, 0, PlainIO, LLIO>(args, 0, l, idx, tk, wl);
                else step_proj<T, kXRmsNorm, KCD, kOutRope, 0, LLIO, LLIO>(args, 0, l, idx, tk, wl);
                break;
            case 1: {
                // Work-group w runs on XCD w % 8, and job j on work-group
                // j % G: jobs whose index agrees mod 8 share an XCD (and its
                // L2).  Give them consecutive query heads, i.e. the heads of
                // one KV head, so that head's cache rows are fetched into
                // one L2 instead of one per query head.
                const int hq = (int)args.hq;
                const int head = (hq % 8 == 0) ? (idx % 8) * (hq / 8) + idx / 8 : idx;
                step_attention<T, HD>(args, l, head, tk);
                break;
            }
            case 2: step_proj<T, kXPlain, KCD, kOutPlain, 0, LLIO, LLIO>(args, 2, l, idx, tk, wl); break;
            case 3: step_proj<T, kXRmsNorm, KCD, kOutSwiGlu, RLD, LLIO, LLIO>(args, 3, l, idx, tk, wl); break;
            case 4: step_proj<T, kXPlain, KCF, kOutPlain, RLF, LLIO, LLIO>(args, 4, l, idx, tk, wl); break;
            case 5:
                step_proj<T, kXRmsNorm, KCD, kOutPlain, RLD, LLIO, CoherentIO>(args, 5, l, idx, tk, wl);
                signal_head(args, idx);
                break;
            case 6:
                step_proj<T, kXRmsNorm, KCD, kOutPlain, 0, LLIO, CoherentIO, kHeadTailRows>(args, 6, l, idx, tk, wl);
                signal_head(args, idx);
                break;
            default: step_sample<T>(args, tk, wl); break;
        }
        // the LDS buffers are free for the next job
        __syncthreads();
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

// The kernel instance for a shape (hd 64 / 128, the K-chunk buckets of d and ffn).
template <typename T, int HD, int KCD>
static const void *step_kernel_kcf(int kcf) {
    switch (kcf) {
        case 4: return reinterpret_cast<const void *>(&decode_step_kernel<T, HD, KCD, 4>);
        case 8: return reinterpret_cast<const void *>(&decode_step_kernel<T, HD, KCD, 8>);
        case 12: return reinterpret_cast<const void *>(&decode_step_kernel<T, HD, KCD, 12>);
        default: return reinterpret_cast<const void *>(&decode_step_kernel<T, HD, KCD, 16>);
    }
}

template <typename T>
static const void *step_kernel(int64_t hd, int kcd, int kcf) {
    if (hd == 64) return kcd == 4 ? step_kernel_kcf<T, 64, 4>(kcf) : step_kernel_kcf<T, 64, 8>(kcf);
    return kcd == 4 ? step_kernel_kcf<T, 128, 4>(kcf) : step_kernel_kcf<T, 128, 8>(kcf);
}

// Keys the one-pass row-wide attention covers: 8 waves x (64 / (hd / 8))
// lane groups x 12 keys per lane (768 at hd 64, 384 at hd 128).  A key past
// that range would be dropped, so larger caches are refused.
static int64_t step_max_keys(int64_t hd) { return (int64_t)kStepWaves * (64 / (hd / 8)) * 12; }

// Whether one work-group of `fn` fits on a CU with nothing else running
// (LDS, registers): the step's jobs wait on each other across work-groups,
// which is only safe when the whole one-per-CU grid is resident at once.
// Queried once per device and kernel instance.
static bool step_resident(const void *fn) {
    static const void *seen_fn[64][32];
    static int seen_ok[64][32];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    for (int i = 0; i < 32; ++i) {
        if (seen_fn[dev][i] == fn) return seen_ok[dev][i] == 1;
        if (!seen_fn[dev][i]) {
            int nb = 0;
            const bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, kStepThreads, 0) == hipSuccess &&
                            nb >= 1;
            seen_ok[dev][i] = ok ? 1 : 2;
            seen_fn[dev][i] = fn;
            return ok;
        }
    }
    return false;
}

}  // namespace kuiops

using namespace kuiops;

// Shape gate of the persistent step (host only, no GPU call); on success the
// K-chunk buckets of d and ffn.
static int step_gate(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv, int64_t hd, int64_t vocab,
                     int64_t cache_cap, int dtype, int &kcd, int &kcf) {
    if (n_layers <= 0 || d <= 0 || ffn <= 0 || hq <= 0 || hkv <= 0 || hd <= 0 || vocab <= 0 || cache_cap <= 0)
        return KUIOPS_E_INVALID;
    if (hq % hkv || hd % 2) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if ((hd != 64 && hd != 128) || d != hq * hd || d % 8 || ffn % 8) return KUIOPS_E_UNSUPPORTED;
    kcd = kc_bucket(d);
    kcf = kc_bucket(ffn);
    if (kcd == 0 || kcd > 8 || kcf == 0) return KUIOPS_E_UNSUPPORTED;   // paired epilogues: d <= 4096
    if (vocab > (int64_t)kSmThreads * kSmCache || vocab > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    if (n_layers > 1024 || cache_cap > step_max_keys(hd)) return KUIOPS_E_UNSUPPORTED;
    return KUIOPS_OK;
}

extern "C" int kuiops_decode_step_supported(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv,
                                            int64_t hd, int64_t vocab, int64_t cache_cap, int dtype) {
    int kcd = 0, kcf = 0;
    const int rc = step_gate(n_layers, d, ffn, hq, hkv, hd, vocab, cache_cap, dtype, kcd, kcf);
    if (rc != KUIOPS_OK) return rc;
    const void *fn = dtype == KUIOPS_BF16 ? step_kernel<bf16_t>(hd, kcd, kcf) : step_kernel<f16_t>(hd, kcd, kcf);
    return step_resident(fn) ? KUIOPS_OK : KUIOPS_E_UNSUPPORTED;
}

// Epoch-tagged scratch vectors, in elements: h0, h1 [d], q, att [hq*hd],
// o [d], act [ffn], down [d], k / v copies [layers][steps][hkv*hd]; two
// elements per 8-byte word, each vector 256-byte aligned.
static size_t step_scratch_layout(int64_t n_layers, int64_t n_steps, int64_t d, int64_t ffn, int64_t hq,
                                  int64_t hkv, int64_t hd, size_t off[9]) {
    const int64_t kv = n_layers * n_steps * hkv * hd;
    const int64_t n[9] = {d, d, hq * hd, hq * hd, d, ffn, d, kv, kv};
    size_t o = 0;
    for (int i = 0; i < 9; ++i) {
        off[i] = o;
        o += (size_t)cdiv(n[i] / 2 * 8, 256) * 256;
    }
    return o;
}

extern "C" size_t kuiops_decode_step_sync_bytes(int64_t n_layers) {
    (void)n_layers;
    return (size_t)(kSubCounters + 3) * kCounterStride * sizeof(unsigned);
}

extern "C" size_t kuiops_decode_step_scratch_bytes(int64_t n_layers, int64_t n_steps, int64_t d, int64_t ffn,
                                                   int64_t hq, int64_t hkv, int64_t hd) {
    if (n_layers <= 0 || n_steps <= 0 || d <= 0 || ffn <= 0 || hq <= 0 || hkv <= 0 || hd <= 0) return 0;
    size_t off[9];
    return step_scratch_layout(n_layers, n_steps, d, ffn, hq, hkv, hd, off);
}

extern "C" int kuiops_decode_step(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv, int64_t hd,
                                  int64_t vocab, int64_t cache_cap, int dtype, float eps,
                                  const kuiops_step_layer *layers, int64_t sk_head, int64_t sk_pos,
                                  int64_t sv_head, int64_t sv_pos, const void *embed, const void *final_norm,
                                  const void *lm_head, const float *inv_freq, int64_t *tok, int32_t *pos,
                                  int32_t *kv_len, int64_t *history, int64_t hist_len, float *prob, void *logits,
                                  int64_t n_steps, void *scratch, size_t scratch_bytes, void *sync,
                                  size_t sync_bytes, void *stream) {
    int kcd = 0, kcf = 0;
    const int gate = step_gate(n_layers, d, ffn, hq, hkv, hd, vocab, cache_cap, dtype, kcd, kcf);
    if (gate != KUIOPS_OK) return gate;
    if (!layers || !embed || !final_norm || !lm_head || !inv_freq || !tok || !pos || !kv_len || !logits ||
        !scratch || !sync)
        return KUIOPS_E_INVALID;
    if (history && hist_len <= 0) return KUIOPS_E_INVALID;
    if (n_steps < 1 || n_steps > kMaxSteps) return KUIOPS_E_UNSUPPORTED;
    size_t off[9];
    if (scratch_bytes < step_scratch_layout(n_layers, n_steps, d, ffn, hq, hkv, hd, off) || !aligned16(scratch))
        return KUIOPS_E_WORKSPACE;
    if (sync_bytes < kuiops_decode_step_sync_bytes(n_layers) || !aligned16(sync)) return KUIOPS_E_WORKSPACE;
    for (const void *p : {embed, final_norm, lm_head, (const void *)logits})
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
    char *sc = reinterpret_cast<char *>(scratch);
    void **vec[9] = {&a.h0, &a.h1, &a.q, &a.att, &a.o, &a.act, &a.down, &a.kf, &a.vf};
    for (int i = 0; i < 9; ++i) *vec[i] = sc + off[i];
    a.logits = logits;
    a.sync = reinterpret_cast<unsigned *>(sync);
    const int64_t rows_d = (int64_t)kStepWaves * rows_per_wave(kcd);
    const int64_t rows_dl = (int64_t)kStepWaves * (rows_per_wave(kcd) + lds_rows_per_wave(kcd));
    const int64_t rows_fl = (int64_t)kStepWaves * (rows_per_wave(kcf) + lds_rows_per_wave(kcf));
    // LM head: at most one full-size job per work-group (their weights load
    // while the last layer runs), the remaining rows in small jobs spread
    // over the grid (a second full-size round would load its weights only
    // after the first)
    const int64_t G = num_cus();
    const int64_t head_a = std::min(cdiv(vocab, rows_dl), G);
    const int64_t split = std::min(vocab, head_a * rows_dl);
    const int64_t nj[kKinds] = {cdiv((hq + 2 * hkv) * hd, rows_d), hq, cdiv(d, rows_d), cdiv(2 * ffn, rows_dl),
                                cdiv(d, rows_fl), head_a, cdiv(vocab - split, (int64_t)kStepWaves * kHeadTailRows), 1};
    a.head_split = split;
    int64_t per_layer = 0;
    for (int k = 0; k < kLayerKinds; ++k) per_layer += nj[k];
    const int64_t per_token = n_layers * per_layer + nj[5] + nj[6] + nj[7];
    const int64_t total = n_steps * per_token;
    if (total > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    for (int k = 0; k < kKinds; ++k) a.njobs[k] = (int)nj[k];
    a.per_layer = (int)per_layer;
    a.per_token = (int)per_token;
    a.steps = (int)n_steps;
    a.total = (int)total;
    // one work-group per CU: all resident at once (a job waits only on jobs
    // with lower indices, which resident work-groups run)
    const dim3 grid((unsigned)G);
    const void *fn = dtype == KUIOPS_BF16 ? step_kernel<bf16_t>(hd, kcd, kcf) : step_kernel<f16_t>(hd, kcd, kcf);
    if (!step_resident(fn)) return KUIOPS_E_UNSUPPORTED;
    void *kargs[] = {&a};
    if (hipLaunchKernel(fn, grid, dim3(kStepThreads), kargs, 0, as_stream(stream)) != hipSuccess) return KUIOPS_E_HIP;
    return launch_status();
}

extern "C" int kuiops_decode_step_error(void *sync, int64_t n_layers, void *stream) {
    (void)n_layers;
    if (!sync) return KUIOPS_E_INVALID;
    unsigned *w = reinterpret_cast<unsigned *>(sync) + kSubCounters * kCounterStride;
    unsigned v = 0;
    hipStream_t st = as_stream(stream);
    if (hipMemcpyAsync(&v, w, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess) return KUIOPS_E_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return KUIOPS_E_HIP;
    if (v && hipMemsetAsync(w, 0, sizeof(unsigned), st) != hipSuccess) return KUIOPS_E_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return KUIOPS_E_HIP;
    return v ? 1 : 0;
}
