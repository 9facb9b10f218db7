// Persistent single-launch decode step.
//
// The whole L = 1 step of src/detail/dense_decoder.cpp:439-496 (run_layers_,
// :526-681, at one token) — embedding, every layer, final norm, lm_head,
// greedy argmax and the token feedback — runs as ONE launch with one
// co-resident workgroup per CU.  Stages that the multi-kernel step separates with a
// kernel boundary are separated here by dataflow: every vector a stage hands
// to the next is written as 64-bit words {16-bit tag, three FP16 values} (or
// {tag, one 32-bit value} for split records and argmax candidates) with
// device-scope relaxed atomic stores, and consumers poll those words
// (device-scope relaxed atomic loads, coherent across XCDs) until every tag
// equals the tag of the (epoch, layer, stage) they wait for.  The polled
// volume is what an all-to-all hand-off costs, hence three values per word.
// The epoch cycles through 1..63; the host re-initializes the words
// (bx_persist_ws_init) before each cycle, so a word never holds a stale tag
// equal to the one awaited.  A poll gives up after a bounded number of rounds
// and raises a shared abort flag that every other poll checks, so all waves
// leave the kernel on any failure.
//
// Per layer (WG w of G):
//   A  rms_norm(h) -> rows of [Wq; Wk; Wv] (segments spread over G by bytes)
//   B  WGs (group g, split s): QK-norm, RoPE, KV-cache write of position pos,
//      split-K attention partial over keys [kb, ke); split 0 of each group
//      combines the partials of its group -> FP16 attention output
//   C  rows of Wo owned by w (H/G rows) + residual kept in the WG's LDS
//   D  rms_norm(h) -> gate/up row pairs -> FP16 silu(g)*u
//   E  rows of Wd owned by w + residual
// Head: rms_norm(h) -> lm_head rows -> FP16 logits + per-WG argmax; WG 0
// reduces the candidates (lowest index on ties) and advances tok/pos.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "gemv_core.h"

namespace bx {
namespace {

constexpr int kPT = 256;            // threads per workgroup
constexpr int kPW = kPT / 64;       // waves
constexpr int kMaxGq = 8;           // query heads per KV head
constexpr int kTile = 128;          // keys per attention tile
constexpr int kMaxOwn = 64;         // residual rows owned per WG
constexpr uint32_t kSpinCheck = 128;        // poll rounds between abort checks
constexpr uint32_t kSpinLimit = 1u << 21;   // poll rounds before giving up (~1 s)
constexpr int kTraceSlots = 1024;          // per WG: 1 + 10 per layer + 4
constexpr int kTraceLayer = 14;            // attention sub-stage stamps (slots 900-907) of this layer

struct PArgs {
    int H, F, n_q, n_kv, hd, V, cap, L;
    float eps;
    int qk_norm;                     // 0: no per-head q/k RMSNorm (q_norm / k_norm not read)
    int g_q, g_k;                    // WGs of the q and k segments of stage A (v gets the rest)
    uint32_t epoch;
    const bx_decode_layer* layers;   // device array of L layers
    const uint16_t* embed;
    const uint16_t* final_norm;
    const void* lm_head;
    const float* cos_t;
    const float* sin_t;
    int32_t* scal;                   // tok, pos, next, count, hist[...]
    uint16_t* logits;
    uint32_t* ctrl;                  // [0] abort flag, [1] failure site
    uint64_t* hbuf;                  // words3(H) words: FP16 residual triples
    uint64_t* qw;                    // n_q * hw words: q triples per head (hw = head_words(hd))
    uint64_t* kw;                    // n_kv * hw words: k triples per head
    uint64_t* vw;                    // n_kv * hw words: v triples per head
    uint64_t* attn;                  // n_q * hw words: attention output triples per head
    uint64_t* act;                   // words3(F) words: SwiGLU output triples
    uint64_t* part;                  // n_kv * part_words_per_group words: FP32 split records
    uint64_t* cand;                  // 2 G words: per-WG argmax value / index
    int64_t part_stride;             // words of split records per KV group
    uint64_t* trace;                 // optional wall-clock stamps [G][kTraceSlots] (bx_persist_trace)
};

// ---- tagged words ----------------------------------------------------------
// bits 48-63: tag; bits 0-47: three FP16 values (v0 at bit 0, v1 at 16, v2 at
// 32) or bits 0-31: one 32-bit value.  tag = (epoch mod 64) << 10 | layer << 3
// | stage with epoch in 1..63 and layer <= 126, so the all-ones pattern the
// words are initialized to is never a live tag.
__host__ __device__ constexpr int words3(int n) { return (n + 2) / 3; }
// Words per head of a per-head triple vector: words3(hd) rounded up to even,
// so every head (and group of heads) starts 16-byte aligned for the paired
// polls; a padding word holds no element but is written and polled like the
// others.
__host__ __device__ constexpr int head_words(int hd) { return (words3(hd) + 1) & ~1; }

// x / d for 0 <= x < 2^16 and 1 <= d <= 2^16 by a multiply-high with
// ceil(2^32 / d): the error x / 2^32 < 2^-16 never crosses an integer, since
// fractional parts of x / d are multiples of 1 / d.  A runtime integer
// division would cost tens of instructions inside a poll loop.
struct FastDiv {
    uint32_t d, m;
    __device__ __forceinline__ explicit FastDiv(int d_)
        : d((uint32_t)d_), m((uint32_t)(0xffffffffu / (uint32_t)d_) + 1u) {}
    __device__ __forceinline__ int div(int x) const { return d == 1 ? x : (int)__umulhi((uint32_t)x, m); }
};

__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 48) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_h3(uint64_t* p, uint32_t tag, uint32_t v0, uint32_t v1, uint32_t v2) {
    __hip_atomic_store(p, ((uint64_t)tag << 48) | ((uint64_t)v2 << 32) | ((uint64_t)v1 << 16) | (uint64_t)v0,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t word_tag(uint64_t w) { return (uint32_t)(w >> 48); }
__device__ __forceinline__ uint32_t word_lo(uint64_t w) { return (uint32_t)w; }
__device__ __forceinline__ uint32_t word_h(uint64_t w, int j) { return (uint32_t)(w >> (16 * j)) & 0xffffu; }
__device__ __forceinline__ uint32_t tag_of(const PArgs& a, int layer, int stage) {
    return ((a.epoch & 63u) << 10) | ((uint32_t)layer << 3) | (uint32_t)stage;
}

// The thread index through an opaque move: values derived from it (per-lane
// addresses) cannot be hoisted out of the layer loop, where dozens of them
// would outlive the register file and spill.
__device__ __forceinline__ int tidx() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

// A zero the compiler cannot see through.  Added to the per-lane address
// terms inside the layer loop, it keeps those addresses from being hoisted
// out of the loop, where dozens of loop-invariant 64-bit addresses would
// outlive the register file and spill.
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return z;
}

// Compiler memory barrier after a prefetch: without it the compiler sinks
// the weight loads to their first use (past the polls in between) and waits
// for them there, so nothing is in flight ahead of time.  It emits no
// instruction and does not wait for the loads.
// Compiler barrier after a batch of LDS reads: keeps the reads issued
// together, ahead of their uses (otherwise each read may be scheduled next to
// its use, one LDS latency per read).
__device__ __forceinline__ void lds_batch() { asm volatile("" ::: "memory"); }

template <int ID>
__device__ __forceinline__ void pin_loads() { asm volatile("; prefetch point %0" ::"i"(ID) : "memory"); }

// Wall-clock stamp of a stage boundary (thread 0) when tracing is on.
__device__ __forceinline__ void stamp(const PArgs& a, int slot) {
    if (a.trace && tidx() == 0) a.trace[(size_t)blockIdx.x * kTraceSlots + slot] = wall_clock64();
}

__device__ __forceinline__ bool aborted(const PArgs& a) {
    return __hip_atomic_load(a.ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void raise_abort(const PArgs& a, uint32_t site) {
    __hip_atomic_store(a.ctrl + 1, site, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.ctrl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll words [0, n) of buf two at a time: 16-byte device-scope loads (sc1
// buffer loads) of word pairs.  Each 8-byte half carries its own tag, so a
// load that saw two different writes cannot pass a stale half.  Thread t owns
// pairs t, t + kPT, ...; E pairs in flight per thread; sink(i, word) for each
// word once its tag matches.  false on abort.
template <int E, class Sink>
__device__ __forceinline__ bool poll_words(const PArgs& a, const uint64_t* buf, int n, uint32_t tag, uint32_t site,
                                           Sink sink) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(buf), 0, (n + 1) / 2 * 16, 0x00020000);
    const int np = (n + 1) / 2;
    for (int base = 0; base < np; base += E * kPT) {
        uint32_t pend = 0;   // bit 2e + h: word h of pair e
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int pi = base + tidx() + e * kPT;
            if (pi < np) pend |= (2 * pi + 1 < n ? 3u : 1u) << (2 * e);
        }
        uint32_t rounds = 0;
        while (pend) {
            u4v v[E];
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (pend & (3u << (2 * e)))
                    v[e] = __builtin_amdgcn_raw_buffer_load_b128(rs, (base + tidx() + e * kPT) * 16, 0, 16);
#pragma unroll
            for (int e = 0; e < E; ++e) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t bit = 1u << (2 * e + h);
                    const uint64_t w = ((uint64_t)v[e][2 * h + 1] << 32) | v[e][2 * h];
                    if ((pend & bit) && word_tag(w) == tag) {
                        pend &= ~bit;
                        sink(2 * (base + tidx() + e * kPT) + h, w);
                    }
                }
            }
            if (pend) {
                ++rounds;
                if (rounds % kSpinCheck == 0) {
                    if (aborted(a)) return false;
                    if (rounds >= kSpinLimit) {
                        raise_abort(a, site);
                        return false;
                    }
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    return true;
}

// Poll np word pairs at base + off(p) (16-byte aligned, both words live),
// E pairs in flight per thread; sink(p, h, word) for word h of pair p once its
// tag matches.  For vectors spread over several buffers of one allocation.
template <int E, class Off, class Sink>
__device__ __forceinline__ bool poll_pairs(const PArgs& a, const uint64_t* base, int np, uint32_t tag, uint32_t site,
                                           Off off, Sink sink) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base), 0, 0x7fffffff,
                                                                        0x00020000);
    for (int b = 0; b < np; b += E * kPT) {
        uint32_t pend = 0;
        int wo[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int pi = b + tidx() + e * kPT;
            wo[e] = pi < np ? off(pi) : 0;
            if (pi < np) pend |= 3u << (2 * e);
        }
        uint32_t rounds = 0;
        while (pend) {
            u4v v[E];
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (pend & (3u << (2 * e))) v[e] = __builtin_amdgcn_raw_buffer_load_b128(rs, wo[e] * 8, 0, 16);
#pragma unroll
            for (int e = 0; e < E; ++e) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t bit = 1u << (2 * e + h);
                    const uint64_t w = ((uint64_t)v[e][2 * h + 1] << 32) | v[e][2 * h];
                    if ((pend & bit) && word_tag(w) == tag) {
                        pend &= ~bit;
                        sink(b + tidx() + e * kPT, h, w);
                    }
                }
            }
            if (pend) {
                ++rounds;
                if (rounds % kSpinCheck == 0) {
                    if (aborted(a)) return false;
                    if (rounds >= kSpinLimit) {
                        raise_abort(a, site);
                        return false;
                    }
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    return true;
}

// ---- LDS arena -------------------------------------------------------------

struct Arena {
    uint32_t* xs;     // swizzled FP16 pairs, Kmax / 2
    float* xsum;      // Kmax / 8 sums of 8 consecutive elements
    float* hv;        // H (full residual for the norms)
    float* own;       // kMaxOwn residual rows owned by this WG
    float* rows;      // kMaxOwn stage outputs of this WG, gathered before they are packed into words
    float* red;       // 64 reduction scratch
    float* att;       // attention scratch (see attention_stage)
};

__host__ __device__ inline size_t att_scratch_bytes(int hd, int Gq);

// LDS bytes of the kernel's copy of the layer table (ahead of the arena).
__host__ __device__ inline size_t layer_table_bytes(int L) {
    return ((size_t)L * sizeof(bx_decode_layer) + 15) / 16 * 16;
}

__host__ __device__ inline size_t arena_bytes(int H, int F, int qd, int hd, int Gq) {
    const int kmax = H > F ? (H > qd ? H : qd) : (F > qd ? F : qd);
    return (size_t)kmax * 2 + (size_t)(kmax / 8) * 4 + (size_t)H * 4 + 2 * kMaxOwn * 4 + 64 * 4 +
           att_scratch_bytes(hd, Gq);
}

__device__ __forceinline__ Arena make_arena(unsigned char* base, int H, int F, int qd) {
    const int kmax = H > F ? (H > qd ? H : qd) : (F > qd ? F : qd);
    Arena r;
    size_t o = 0;
    r.xs = reinterpret_cast<uint32_t*>(base + o); o += (size_t)kmax * 2;
    r.xsum = reinterpret_cast<float*>(base + o); o += (size_t)(kmax / 8) * 4;
    r.hv = reinterpret_cast<float*>(base + o); o += (size_t)H * 4;
    r.own = reinterpret_cast<float*>(base + o); o += kMaxOwn * 4;
    r.rows = reinterpret_cast<float*>(base + o); o += kMaxOwn * 4;
    r.red = reinterpret_cast<float*>(base + o); o += 64 * 4;
    r.att = reinterpret_cast<float*>(base + o);
    return r;
}

// A norm's FP16 gamma for the 8-element chunks c = tidx() + j kPT, loaded
// into registers before the normalized vector's input arrives.
constexpr int kGammaChunks = 2;   // hidden <= 2 * 8 * kPT
struct GammaRegs {
    u4v v[kGammaChunks];
    __device__ __forceinline__ void load(const void* gamma, int K) {
#pragma unroll
        for (int j = 0; j < kGammaChunks; ++j) {
            const int c = tidx() + j * kPT;
            if (8 * c < K) v[j] = gptr<u4v>(gamma)[c];
        }
    }
};
// One FP16 value (bits v) of element e into the swizzled LDS pairs: group
// g = e / 4 holds dwords 2g = (x0, x2) and 2g + 1 = (x1, x3).
__device__ __forceinline__ void put_swz(uint32_t* xs, int e, uint32_t v) {
    reinterpret_cast<uint16_t*>(xs)[4 * (e >> 2) + 2 * (e & 1) + ((e >> 1) & 1)] = (uint16_t)v;
}

// Poll nw words of FP16 triples into the swizzled activation of K elements
// (element of word i, slot j: elem(i, j), skipped when >= K), then the
// 8-element sums.  E words in flight per thread.
template <int E, class Elem>
__device__ __forceinline__ bool poll_triples_to_xs(const PArgs& a, const Arena& ar, const uint64_t* buf, int nw, int K,
                                                   uint32_t tag, uint32_t site, Elem elem) {
    const bool ok = poll_words<E>(a, buf, nw, tag, site, [&](int i, uint64_t w) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int e = elem(i, j);
            if (e >= 0) put_swz(ar.xs, e, word_h(w, j));
        }
    });
    if (!__syncthreads_and(ok)) return false;
    sums8_from_lds(ar.xs, K, ar.xsum);
    __syncthreads();
    return true;
}

// Element of slot j of word i in a per-head triple layout (hw words per head
// of HD elements); -1 for the padding slots at a head's end.
template <int HD>
__device__ __forceinline__ int head_elem(int i, int j) {
    constexpr int hw = head_words(HD);
    const int h = i / hw, d = 3 * (i - h * hw) + j;
    return d < HD ? h * HD + d : -1;
}

// First row of word W in a per-head triple layout (rows of a head are
// contiguous; words never straddle heads; a padding word starts at the next
// head's first row and holds none).
template <int HD>
__device__ __forceinline__ int head_row(int W) {
    constexpr int hw = head_words(HD);
    return (W / hw) * HD + min(3 * (W % hw), HD);
}

// Pack this WG's stage outputs (src[r - r0] for rows r of words [wb, we),
// gathered in LDS) into FP16 triples and store them.  row(W) is the first row of
// word W, nrows(W) its count (<= 3).
template <class Row, class NRows>
__device__ __forceinline__ void emit_triples(const float* src, uint64_t* out, int wb, int we, int r0, uint32_t tag,
                                             Row row, NRows nrows) {
    for (int W = wb + tidx(); W < we; W += kPT) {
        const int r = row(W) - r0, n = nrows(W);
        const uint32_t v0 = n > 0 ? f2h(src[r]) : 0u;
        const uint32_t v1 = n > 1 ? f2h(src[r + 1]) : 0u;
        const uint32_t v2 = n > 2 ? f2h(src[r + 2]) : 0u;
        st_h3(out + W, tag, v0, v1, v2);
    }
}

// R rows x UPL units of one matrix held in a wave's registers: loaded ahead
// of the activation they meet (the weights do not depend on it), dotted later.
template <int FMT, int UPL, int R>
struct RowBlock {
    typename RawOf<FMT>::T raw[R][UPL];

    // Every load is issued unconditionally (rows and units clamped into the
    // matrix, the extras ignored by dot): the compiler then counts the loads in
    // flight exactly and waits only for the ones a later use needs, not for
    // loads issued after these.
    __device__ __forceinline__ void load(const void* W, int64_t N, int K, int64_t row0) {
        const int lane = tidx() & 63;
        const int U = K / 32;
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            int64_t row = row0 + rr < N ? row0 + rr : N - 1;
            if (row < 0) row = 0;
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = lane + 64 * i;
                raw[rr][i] = load_unit<FMT>(W, N, K, row, u < U ? u : U - 1);
            }
        }
    }

    __device__ __forceinline__ void dot(int K, const XCache<FMT, UPL>& xu, float (&out)[R]) const {
        const int lane = tidx() & 63;
        const int U = K / 32;
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                // a select, not a branch: no control flow between the loads and the math
                const int u = lane + 64 * i;
                const int uc = u < U ? u : U - 1;
                const float c = dot_reg(raw[rr][i], uc, xu.get(i, uc));
                acc += u < U ? c : 0.f;
            }
            out[rr] = acc;
        }
        wave_sum_n<R>(out);
    }
};

// A wave's row tasks first, first + stride, ... below end: the first task's
// block was loaded ahead by the caller, later ones load in place.  The first
// task is peeled off the loop so that no in-loop load merges into its path:
// its wait then covers its own loads and the ones issued before them, not the
// next stage's blocks requested after it.
template <class Load, class Comp>
__device__ __forceinline__ void peeled_tasks(int first, int end, int stride, Load&& load, Comp&& comp) {
    if (first < end) {
        comp(first);
        for (int r = first + stride; r < end; r += stride) {
            load(r);
            comp(r);
        }
    }
}

// The same tasks with two blocks in turn: b0 holds the first task (loaded by
// the caller), and every task but the last requests the next task's block into
// the other one before its own math, so a wave with several tasks waits for
// memory once.  Each path issues its loads unconditionally, so the compiler's
// wait before a task's math covers that task's loads and not the ones requested
// after them; a single task takes the path with no loads, as peeled_tasks.
template <class Blk, class Load, class Comp>
__device__ __forceinline__ void piped_tasks(Blk& b0, Blk& b1, int first, int end, int stride, Load&& load,
                                            Comp&& comp) {
    for (int t = first; t < end;) {
        if (t + stride >= end) {
            comp(b0, t);
            break;
        }
        load(b1, t + stride);
        comp(b0, t);
        t += stride;
        if (t + stride >= end) {
            comp(b1, t);
            break;
        }
        load(b0, t + stride);
        comp(b1, t);
        t += stride;
    }
}

// Rows [r0, r1) of W (N x K): wave w takes tasks of R rows starting at
// r0 + w R with stride kPW R.  prefetch() loads the first task before the
// caller waits for the activation; finish() computes every task (later tasks
// load in turn) and calls epi(row, value) on lane 0.
template <int FMT, int UPL, int R>
struct WgRows {
    RowBlock<FMT, UPL, R> blk;
    int first;

    __device__ __forceinline__ void prefetch(const void* W, int64_t N, int K, int r0, int r1) {
        first = r0 + (int)(tidx() >> 6) * R;
        if (first < r1) blk.load(W, N, K, first);
    }

    template <class Epi>
    __device__ __forceinline__ void finish(const void* W, int64_t N, int K, int r1, const Arena& ar, Epi epi) {
        if (first >= r1) return;
        const int lane = tidx() & 63;
        XCache<FMT, UPL> xu;
        xu.init(ar.xs, ar.xsum, K);
        for (int t = first; t < r1; t += kPW * R) {
            if (t != first) blk.load(W, N, K, t);
            float o[R];
            blk.dot(K, xu, o);
            if (lane == 0) {
#pragma unroll
                for (int rr = 0; rr < R; ++rr)
                    if (t + rr < r1) epi(t + rr, o[rr]);
            }
        }
    }
};

// lm_head rows [r0, r1) with NB blocks in turn: while a task's math runs,
// the next NB - 1 tasks' loads are in flight (a wave's tasks are r0 + wave R,
// then every kPW R rows).  The caller loads b[0]; the requests are
// unconditional, a task past the range re-reading the range's last rows, so
// the compiler's wait before each task's math counts exactly the loads issued
// after it.
template <int FMT, int UPL, int R, int NB, class Epi>
__device__ __forceinline__ void head_rows_nb(RowBlock<FMT, UPL, R> (&b)[NB], const void* W, int64_t N, int K,
                                             int r0, int r1, const Arena& ar, Epi epi) {
    const int lane = tidx() & 63;
    const int step = kPW * R;
    const int t0 = r0 + (int)(tidx() >> 6) * R;
    auto at = [&](int t) { return t < r1 ? t : (r1 - R > r0 ? r1 - R : r0); };
#pragma unroll
    for (int j = 1; j < NB - 1; ++j) b[j].load(W, N, K, at(t0 + j * step));
    XCache<FMT, UPL> xu;
    xu.init(ar.xs, ar.xsum, K);
    for (int t = t0; t < r1; t += NB * step) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int tj = t + j * step;
            if (tj >= r1) return;
            b[(j + NB - 1) % NB].load(W, N, K, at(tj + (NB - 1) * step));
            float o[R];
            b[j].dot(K, xu, o);
            if (lane == 0) {
#pragma unroll
                for (int rr = 0; rr < R; ++rr)
                    if (tj + rr < r1) epi(tj + rr, o[rr]);
            }
        }
    }
}

__device__ __forceinline__ void range_of(int n, int parts, int i, int& b, int& e) {
    b = (int)((int64_t)n * i / parts);
    e = (int)((int64_t)n * (i + 1) / parts);
}

// ---- attention (stage B) ---------------------------------------------------

// Keys per split and split count for context length n: splits <= smax, keys
// a multiple of kSplitQ (short splits keep each workgroup's chain short).
constexpr int kSplitQ = 16;
__device__ __forceinline__ void split_plan(int n, int smax, int& kps, int& S) {
    kps = (n + smax - 1) / smax;
    kps = (kps + kSplitQ - 1) / kSplitQ * kSplitQ;
    if (kps < kSplitQ) kps = kSplitQ;
    S = (n + kps - 1) / kps;
}

// Output words each of a group's combining WGs merges per head: wpc words =
// dsl = 3 wpc head dims, so a combiner emits whole FP16 triples; ncomb =
// ceil(head_words(hd) / wpc) <= S combiners.  A split record holds dsl
// partial sums, m and l, padded to an even word count (paired polls).
__host__ __device__ inline int comb_words(int hd, int S) { return (head_words(hd) + S - 1) / S; }
__host__ __device__ inline int rec_words(int wpc) { return (3 * wpc + 2 + 1) & ~1; }

// Attention scratch inside the arena (host and device agree on this size):
// the key and value tiles, the group's raw q / k / v rows, and per wave its
// roped q heads (at most two), the current key and value rows, and the
// scores and probabilities of its keys.
__host__ __device__ inline size_t att_wave_floats(int hd) { return (size_t)2 * hd + hd + 2 * kTile; }
__host__ __device__ inline size_t att_scratch_bytes(int hd, int Gq) {
    return (size_t)2 * kTile * hd * 2 + (size_t)(Gq + 2) * hd * 4 + (size_t)kPW * att_wave_floats(hd) * 4;
}
// Key parts per head and heads per wave of the attention stage: the waves
// split the key range of a split (P parts) when there are fewer heads than
// waves, else take HPW heads each.
__host__ __device__ inline int att_parts(int Gq) { return Gq >= kPW ? 1 : kPW / Gq; }
__host__ __device__ inline int att_heads_per_wave(int Gq) { return Gq > kPW ? Gq / kPW : 1; }

template <int HD>
struct AttScratch {
    uint16_t* kt;   // kTile x HD, 16-byte chunks XOR-swizzled by the key
    uint16_t* vt;   // kTile x HD
    float* qraw;    // Gq x HD
    float* kraw;    // HD
    float* vraw;    // HD
    float* wv;      // this wave's area
    __device__ __forceinline__ AttScratch(const Arena& ar, int Gq) {
        kt = reinterpret_cast<uint16_t*>(ar.att);
        vt = kt + kTile * HD;
        qraw = reinterpret_cast<float*>(vt + kTile * HD);
        kraw = qraw + Gq * HD;
        vraw = kraw + HD;
        wv = vraw + HD + (tidx() >> 6) * att_wave_floats(HD);
    }
    // wave area: q16 [2 x HD/2 pairs] | kcur [HD/2] | vcur [HD/2] | sw [kTile] | pw [kTile]
    __device__ __forceinline__ uint32_t* q16(int hh) const { return reinterpret_cast<uint32_t*>(wv) + hh * (HD / 2); }
    __device__ __forceinline__ uint32_t* kcur() const { return reinterpret_cast<uint32_t*>(wv) + HD; }
    __device__ __forceinline__ uint32_t* vcur() const { return kcur() + HD / 2; }
    __device__ __forceinline__ float* sw() const { return wv + 2 * HD; }
    __device__ __forceinline__ float* pw() const { return sw() + kTile; }
};

// HBM -> LDS copies (global_load_lds_dwordx4): lane L of a wave writes the 16
// bytes at its own source address to lds_base + 16 L.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// Keys [c0, c0 + nk) of one KV head into LDS: K with its 16-byte chunks XOR-
// swizzled by the key (chunk d8 of key j at position d8 ^ (j mod HD/8), so
// lanes reading consecutive keys hit distinct banks), V in natural order.
// Slots past nk in the last copy repeat key nk - 1 (in bounds, finite).
template <int HD>
__device__ __forceinline__ void dma_tile(const uint16_t* Kc, const uint16_t* Vc, int64_t kvd, int64_t krow0, int c0,
                                         int nk, uint16_t* kt, uint16_t* vt) {
    constexpr int CPK = HD / 8;
    const int ninst = (nk * CPK + 63) / 64;
    const int wave = tidx() >> 6, lane = tidx() & 63;
    for (int i = wave; i < ninst; i += kPW) {
        const int slot = 64 * i + lane;
        int j = slot / CPK;
        const int pc = slot % CPK;
        if (j >= nk) j = nk - 1;
        const int64_t row = (int64_t)(c0 + j) * kvd + krow0;
        dma16(Kc + row + 8 * (pc ^ (j & (CPK - 1))), kt + 512 * i);
        dma16(Vc + row + 8 * pc, vt + 512 * i);
    }
}

// Words of the split records per KV group, for the largest of any S <= smax:
// ncomb slices x S P partials (P key parts per split) x Gq heads x (dsl
// partial sums + m + l).
inline size_t part_words_per_group(int hd, int Gq, int smax) {
    size_t best = 0;
    for (int S = 1; S <= smax; ++S) {
        const int wpc = comb_words(hd, S), ncomb = (head_words(hd) + wpc - 1) / wpc;
        const size_t n = (size_t)ncomb * S * att_parts(Gq) * Gq * rec_words(wpc);
        if (n > best) best = n;
    }
    return best;
}
// LDS floats a combiner needs: S P x Gq records of dsl + 2 and Gq x S P weights.
inline size_t comb_lds_floats(int hd, int Gq, int smax) {
    size_t best = 0;
    for (int S = 1; S <= smax; ++S) {
        const size_t Sp = (size_t)S * att_parts(Gq);
        const size_t n = Sp * Gq * rec_words(comb_words(hd, S)) + (size_t)Gq * Sp;
        if (n > best) best = n;
    }
    return best;
}

// Per-lane static vectors of one head row (pairs p = lane + 64 i): q_norm and
// k_norm gamma pairs, RoPE cos / sin of row pos.  Loaded before q is ready.
template <int HD>
struct RopeRegs {
    static constexpr int kP = (HD / 2 + 63) / 64;
    uint32_t qg[kP], kg[kP];
    float c[kP], s[kP];
    __device__ __forceinline__ void load(const bx_decode_layer& Ly, const float* cos_row, const float* sin_row,
                                         bool qk_norm) {
        const int lane = tidx() & 63;
#pragma unroll
        for (int i = 0; i < kP; ++i) {
            const int p = lane + 64 * i;
            qg[i] = kg[i] = 0u;
            if (p < HD / 2) {
                if (qk_norm) {
                    qg[i] = gptr<uint32_t>(Ly.q_norm)[p];
                    kg[i] = gptr<uint32_t>(Ly.k_norm)[p];
                }
                c[i] = gptr<float>(cos_row)[p];
                s[i] = gptr<float>(sin_row)[p];
            }
        }
    }
};

__device__ __forceinline__ float r16(float x) { return h2f(f2h(x)); }
__device__ __forceinline__ uint32_t pack16(float lo, float hi) {
    return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}

// RMSNorm of one HD-long FP32 head (one wave) with gamma pairs gm, RoPE with
// the lane's cos/sin, FP16 rounding after each step as the op path stores
// them (q/k-norm into FP16, RoPE in place on FP16) -> FP16 pairs at dst.
// Without QK-norm (qk_norm false) the head is the projection output rounded
// to FP16, then rotated.
template <int HD>
__device__ __forceinline__ void norm_rope_head(const float* src, const uint32_t (&gm)[RopeRegs<HD>::kP],
                                               const RopeRegs<HD>& rr, float eps, bool qk_norm, uint32_t* dst) {
    const int lane = tidx() & 63;
    constexpr int kP = RopeRegs<HD>::kP;
    float x0[kP], x1[kP];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kP; ++i) {
        const int p = lane + 64 * i;
        x0[i] = x1[i] = 0.f;
        if (p < HD / 2) {
            x0[i] = src[2 * p];
            x1[i] = src[2 * p + 1];
            ss += x0[i] * x0[i] + x1[i] * x1[i];
        }
    }
    float inv = 1.0f;
    if (qk_norm) {
        ss = wave_allsum(ss);
        inv = 1.0f / sqrtf(ss / (float)HD + eps);
    }
#pragma unroll
    for (int i = 0; i < kP; ++i) {
        const int p = lane + 64 * i;
        if (p < HD / 2) {
            const float a0 = qk_norm ? r16(x0[i] * inv * h2f(gm[i] & 0xffff)) : r16(x0[i]);
            const float a1 = qk_norm ? r16(x1[i] * inv * h2f(gm[i] >> 16)) : r16(x1[i]);
            dst[p] = pack16(a0 * rr.c[i] - a1 * rr.s[i], a0 * rr.s[i] + a1 * rr.c[i]);
        }
    }
}

// The first tile of cached keys / values of this workgroup's attention split
// (rows below pos, written by earlier steps) goes straight to LDS.  Issued
// right after the previous stage's output stores, so the copy overlaps the
// wait for q / k / v; nothing touches the tile region until stage B.
template <int HD>
__device__ __forceinline__ void attn_tile_prefetch(const PArgs& a, const Arena& ar, const bx_decode_layer& Ly,
                                                   int pos, int zl) {
    const int G = gridDim.x, w = blockIdx.x;
    const int kvd = a.n_kv * HD;
    const int smax = G / a.n_kv;
    const int g = w % a.n_kv, s = w / a.n_kv;
    if (s >= smax) return;
    int kps, S;
    split_plan(pos + 1, smax, kps, S);
    if (s >= S) return;
    const int kb = s * kps + zl, ke = min(pos + 1, kb + kps);
    uint16_t* kt = reinterpret_cast<uint16_t*>(ar.att);
    dma_tile<HD>(static_cast<const uint16_t*>(Ly.Kc), static_cast<const uint16_t*>(Ly.Vc), kvd, (int64_t)g * HD, kb,
                 ke - kb, kt, kt + kTile * HD);
}

// Stage B for (KV group g, split s) = (w % n_kv, w / n_kv), keys [kb, ke) of
// the split in one LDS tile (the host keeps the cache within smax tiles).
// Every wave works alone on P key parts x HPW heads: q-norm + RoPE of its
// heads, the current key / value (the part holding pos), scores by v_dot2
// with four lanes per key, its own softmax (running max and sum of its keys
// only), P.V with two head dims per lane, and a partial record [o, m, l] per
// (split, part, head).  One barrier (the polled q / k / v and the tile) for
// the whole computation.  Split c < ncomb then merges slice c of all S P
// partials of its group and writes those dims of the FP16 attention output.
template <int HD>
__device__ __forceinline__ bool attention_stage(const PArgs& a, const Arena& ar, const bx_decode_layer& Ly,
                                                int layer, int pos, int zl) {
    constexpr int CPK = HD / 8;     // 16-byte chunks per key row
    constexpr int QC = CPK / 4;     // chunks per lane of a four-lane key dot
    constexpr int hw = head_words(HD);
    const int G = gridDim.x, w = blockIdx.x;
    const int Gq = a.n_q / a.n_kv, kvd = a.n_kv * HD;
    const int smax = G / a.n_kv;
    const int g = w % a.n_kv, s = w / a.n_kv;
    if (s >= smax) return true;
    int kps, S;
    split_plan(pos + 1, smax, kps, S);
    if (s >= S) return true;
    const int kb = s * kps + zl, ke = min(pos + 1, kb + kps);
    const bool has_cur = ke == pos + 1;
    const int wave = tidx() >> 6, lane = tidx() & 63;
    const uint32_t tin = tag_of(a, layer, 0), tout = tag_of(a, layer, 1);
    const int P = att_parts(Gq), HPW = att_heads_per_wave(Gq), Sp = S * P;
    const int part = wave % P, h0 = (wave / P) * HPW;
    const int nk = ke - kb, kpp = (nk + P - 1) / P;
    const int jb = min(nk, part * kpp), je = min(nk, jb + kpp);   // this wave's tile rows
    const int jcur = pos - kb;                                      // tile row of pos when has_cur
    const bool mine_cur = has_cur && jcur >= jb && jcur < je;
    const AttScratch<HD> sc(ar, Gq);
    if (layer == kTraceLayer) stamp(a, 900 + 0);
    RopeRegs<HD> rr;
    rr.load(Ly, a.cos_t + (int64_t)pos * (HD / 2), a.sin_t + (int64_t)pos * (HD / 2), a.qk_norm != 0);
    if (layer == kTraceLayer) stamp(a, 900 + 1);

    // one poll over the group's q words and, for the split holding pos, its k
    // and v words (pairs: hw is even); word offsets from a.qw.  Each wave's
    // polls complete after its own tile copies (in-order counters).
    auto unpack = [](float* dst, int i, uint64_t wd) {
        const int h = i / hw, d = 3 * (i - h * hw);
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if (d + j < HD) dst[h * HD + d + j] = h2f(word_h(wd, j));
    };
    const int npq = Gq * hw / 2, npk = has_cur ? hw / 2 : 0;
    const int kofs = (int)(a.kw - a.qw) + g * hw, vofs = (int)(a.vw - a.qw) + g * hw;
    bool ok = poll_pairs<1>(
        a, a.qw + zl, npq + 2 * npk, tin, 10,
        [&](int p) {
            return p < npq ? g * Gq * hw + 2 * p : (p < npq + npk ? kofs + 2 * (p - npq) : vofs + 2 * (p - npq - npk));
        },
        [&](int p, int h, uint64_t wd) {
            if (p < npq) unpack(sc.qraw, 2 * p + h, wd);
            else if (p < npq + npk) unpack(sc.kraw, 2 * (p - npq) + h, wd);
            else unpack(sc.vraw, 2 * (p - npq - npk) + h, wd);
        });
    __builtin_amdgcn_s_waitcnt(0);   // tile copies of this wave landed (also without polls)
    if (!__syncthreads_and(ok)) return false;
    if (layer == kTraceLayer) stamp(a, 900 + 2);

    // ---- from here each wave works alone
    for (int hh = 0; hh < HPW; ++hh) norm_rope_head<HD>(sc.qraw + (h0 + hh) * HD, rr.qg, rr, a.eps, a.qk_norm != 0, sc.q16(hh));
    if (mine_cur) {
        uint32_t* kc = sc.kcur();
        uint32_t* vc = sc.vcur();
        norm_rope_head<HD>(sc.kraw, rr.kg, rr, a.eps, a.qk_norm != 0, kc);
        for (int p = lane; p < HD / 2; p += 64) vc[p] = pack16(sc.vraw[2 * p], sc.vraw[2 * p + 1]);
        // the current row replaces the stale cache row pos in the tile (another
        // wave of this part writes the same bytes)
        for (int d8 = lane; d8 < CPK; d8 += 64) {
            *reinterpret_cast<u4v*>(sc.kt + jcur * HD + 8 * (d8 ^ (jcur & (CPK - 1)))) =
                *reinterpret_cast<const u4v*>(kc + 4 * d8);
            *reinterpret_cast<u4v*>(sc.vt + jcur * HD + 8 * d8) = *reinterpret_cast<const u4v*>(vc + 4 * d8);
        }
        // KV-cache row pos: once per group
        if (h0 == 0) {
            uint16_t* Kw = static_cast<uint16_t*>(Ly.Kc);
            uint16_t* Vw = static_cast<uint16_t*>(Ly.Vc);
            const int64_t krow0 = (int64_t)g * HD;
            for (int p = lane; p < HD / 2; p += 64) {
                gptr_w<uint32_t>(Kw + (int64_t)pos * kvd + krow0)[p] = kc[p];
                gptr_w<uint32_t>(Vw + (int64_t)pos * kvd + krow0)[p] = vc[p];
            }
        }
    }
    if (layer == kTraceLayer) stamp(a, 900 + 3);

    const float scale = 1.0f / sqrtf((float)HD);
    const int wpc = comb_words(HD, S), dsl = 3 * wpc, ncomb = (hw + wpc - 1) / wpc, rec = rec_words(wpc);
    uint64_t* gbase = a.part + zl + (int64_t)g * a.part_stride;
    auto rec_at = [&](int c, int t, int h) { return gbase + ((int64_t)(c * Sp + t) * Gq + h) * rec; };
    const int nkw = je - jb;   // <= kTile: lane t owns keys jb + t and jb + 64 + t
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = h0 + hh;
        // scores: one lane per key, the whole head dim (q broadcast from LDS,
        // the key row swizzled so that lanes hit distinct banks)
        const uint32_t* q = sc.q16(hh);
        float sv[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int t = lane + 64 * hb;
            sv[hb] = -INFINITY;
            if (64 * hb < nkw) {   // uniform
                const int jr = jb + (t < nkw ? t : nkw - 1);
                const uint16_t* kr = sc.kt + jr * HD;
                float acc = 0.f, acc2 = 0.f;
                // batches of eight chunks: all sixteen LDS reads issued before
                // the math (the barrier keeps the compiler from pairing each
                // read with its use, which would expose every LDS latency)
#pragma unroll
                for (int d0 = 0; d0 < CPK; d0 += 8) {
                    u4v kk[8], qv[8];
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        kk[c] = *reinterpret_cast<const u4v*>(kr + 8 * ((d0 + c) ^ (jr & (CPK - 1))));
                        qv[c] = *reinterpret_cast<const u4v*>(q + 4 * (d0 + c));
                    }
                    lds_batch();
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        acc = dot2(qv[c].x, kk[c].x, acc);
                        acc2 = dot2(qv[c].y, kk[c].y, acc2);
                        acc = dot2(qv[c].z, kk[c].z, acc);
                        acc2 = dot2(qv[c].w, kk[c].w, acc2);
                    }
                }
                if (t < nkw) sv[hb] = (acc + acc2) * scale;
            }
        }
        if (layer == kTraceLayer && hh == 0) stamp(a, 900 + 4);
        // softmax over this wave's keys, in registers (its own max and sum: the
        // combiner rescales the partials)
        const float M = wave_max(fmaxf(sv[0], sv[1]));
        float pv[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) pv[hb] = lane + 64 * hb < nkw ? r16(__expf(sv[hb] - M)) : 0.f;
        const float L = wave_allsum(pv[0] + pv[1]);
        // P.V: lane holds head dims 2 lane, 2 lane + 1; the value rows come in
        // batches of eight LDS reads, the probabilities through the wave's LDS
        // area, four per broadcast read (a readlane per key costs the wait
        // states before its scalar result can feed the multiply; the wave's
        // own LDS writes complete before its later reads)
        float* pw = sc.pw();
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
            if (lane + 64 * hb < nkw) pw[lane + 64 * hb] = pv[hb];
        float o0 = 0.f, o1 = 0.f;
        const uint16_t* vcol = sc.vt + jb * HD + 2 * (2 * lane < HD ? lane : 0);
        for (int t0 = 0; t0 < nkw; t0 += 8) {
            uint32_t vv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int t = min(t0 + u, nkw - 1);
                vv[u] = *reinterpret_cast<const uint32_t*>(vcol + t * HD);
            }
            const u4v pa = *reinterpret_cast<const u4v*>(pw + t0), pc = *reinterpret_cast<const u4v*>(pw + t0 + 4);
            lds_batch();
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float p = t0 + u < nkw ? __uint_as_float(u < 4 ? pa[u] : pc[u - 4]) : 0.f;
                o0 += p * h2f(vv[u] & 0xffff);
                o1 += p * h2f(vv[u] >> 16);
            }
        }
        const int t = s * P + part;
        if (layer == kTraceLayer && hh == 0) stamp(a, 908);
        if (2 * lane < HD) {
            // partial record of (split s, part, head h), in ncomb slices of dsl dims
            const int d = 2 * lane, c0 = d / dsl, c1 = (d + 1) / dsl;
            st_u32(rec_at(c0, t, h) + (d - c0 * dsl), tout, __float_as_uint(o0));
            st_u32(rec_at(c1, t, h) + (d + 1 - c1 * dsl), tout, __float_as_uint(o1));
        }
        for (int c = lane; c < ncomb; c += 64) {
            uint64_t* r = rec_at(c, t, h);
            st_u32(r + dsl, tout, __float_as_uint(M));
            st_u32(r + dsl + 1, tout, __float_as_uint(L));
            if (rec > dsl + 2) st_u32(r + dsl + 2, tout, 0u);
            // the last slice may hold fewer than dsl dims: its unused slots are still
            // polled by the combiner, so they carry the tag too
            for (int dd = max(0, HD - c * dsl); dd < dsl; ++dd) st_u32(r + dd, tout, 0u);
        }
    }
    if (layer == kTraceLayer) stamp(a, 900 + 5);
    if (s >= ncomb) return true;

    // combiner s: dims [s dsl, s dsl + dsl) of every head of the group, over
    // the S P partials (<= 128).  Records transposed in LDS, recs[j N + t Gq +
    // h] (N = S P Gq), so lanes that walk partials read consecutive words.
    __syncthreads();
    float* recs = ar.att;   // S P Gq rec floats (checked on the host)
    const int N = Sp * Gq;
    const uint64_t* mine = gbase + (int64_t)s * Sp * Gq * rec;
    const FastDiv drec(rec);
    ok = poll_words<2>(a, mine, N * rec, tout, 13, [&](int i, uint64_t v) {
        const int r = drec.div(i);
        recs[(i - r * rec) * N + r] = __uint_as_float(word_lo(v));
    });
    if (layer == kTraceLayer) stamp(a, 900 + 6);
    if (!__syncthreads_and(ok)) return false;
    // one wave per (head, third of the slice's words): the partial weights
    // exp(m_t - M) / L with partials over lanes, then one wave sum per dim
    // output words [s wpc, s wpc + nws) of every head of the group
    const int nws = min(wpc, hw - s * wpc);
    for (int job = wave; job < Gq * 3; job += kPW) {
        const int h = job % Gq, third = job / Gq;
        const int kb3 = nws * third / 3, ke3 = nws * (third + 1) / 3;
        if (kb3 >= ke3) continue;   // uniform
        float mt[2], wt[2], lt[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int t = lane + 64 * hb;
            mt[hb] = t < Sp ? recs[dsl * N + t * Gq + h] : -INFINITY;
            lt[hb] = t < Sp ? recs[(dsl + 1) * N + t * Gq + h] : 0.f;
        }
        lds_batch();
        const float M = wave_max(fmaxf(mt[0], mt[1]));
        float lsum = 0.f;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int t = lane + 64 * hb;
            wt[hb] = mt[hb] == -INFINITY ? 0.f : __expf(mt[hb] - M);
            if (t < Sp) lsum += wt[hb] * lt[hb];
        }
        lsum = wave_allsum(lsum);
        const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
        for (int k = kb3; k < ke3; ++k) {
            float ov[3][2];
#pragma unroll
            for (int j = 0; j < 3; ++j)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    const int t = lane + 64 * hb;
                    ov[j][hb] = t < Sp ? recs[(3 * k + j) * N + t * Gq + h] : 0.f;
                }
            lds_batch();
            float acc[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[j] = wt[0] * ov[j][0] + wt[1] * ov[j][1];
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[j] = wave_allsum(acc[j]) * inv;
            if (lane == 0)
                st_h3(a.attn + zl + (int64_t)(g * Gq + h) * hw + s * wpc + k, tout, f2h(acc[0]), f2h(acc[1]),
                      f2h(acc[2]));
        }
    }
    if (layer == kTraceLayer) stamp(a, 900 + 7);
    return true;
}

// ---- the kernel ---------------------------------------------------------------

// Residual poll (FP16 triples into hv) fused with RMSNorm into the swizzled
// FP16 pairs and 8-sums of the dot stages.  hbuf == nullptr: hv already holds
// the residual (layer 0).  Each thread reads back the words it polled itself,
// in a fixed order, for its partial sum of squares, so one barrier serves both
// the all-arrived check and the reduction; each thread then converts 8-element
// chunks c = tidx() + j kPT.
__device__ __forceinline__ bool poll_norm(const PArgs& a, const Arena& ar, const uint64_t* hbuf, uint32_t tag,
                                          uint32_t site, const GammaRegs& gam, float eps) {
    const int K = a.H, nw = words3(K);
    bool ok = true;
    if (hbuf)
        ok = poll_words<2>(a, hbuf, nw, tag, site, [&](int i, uint64_t w) {
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (3 * i + j < K) ar.hv[3 * i + j] = h2f(word_h(w, j));
        });
    // the words this thread polled (pairs tidx() + m kPT), in a fixed order (a
    // deterministic sum, and no read of another thread's words before the barrier)
    float ss = 0.f;
    for (int i = 2 * tidx(); i < nw; i += 2 * kPT) {
#pragma unroll
        for (int j = 0; j < 6; ++j)
            if (3 * i + j < K) ss += ar.hv[3 * i + j] * ar.hv[3 * i + j];
    }
    ss = wave_allsum(ss);
    if ((tidx() & 63) == 0) ar.red[tidx() >> 6] = ss;
    if (!__syncthreads_and(ok)) return false;
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kPW; ++i) tot += ar.red[i];
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
    for (int j = 0; j < kGammaChunks; ++j) {
        const int c = tidx() + j * kPT;
        if (8 * c < K) {
            const float4 v0 = *reinterpret_cast<const float4*>(ar.hv + 8 * c);
            const float4 v1 = *reinterpret_cast<const float4*>(ar.hv + 8 * c + 4);
            const u4v gm = gam.v[j];
            const uint32_t h0 = f2h(v0.x * inv * h2f(gm.x & 0xffff)), h1 = f2h(v0.y * inv * h2f(gm.x >> 16));
            const uint32_t h2 = f2h(v0.z * inv * h2f(gm.y & 0xffff)), h3 = f2h(v0.w * inv * h2f(gm.y >> 16));
            const uint32_t h4 = f2h(v1.x * inv * h2f(gm.z & 0xffff)), h5 = f2h(v1.y * inv * h2f(gm.z >> 16));
            const uint32_t h6 = f2h(v1.z * inv * h2f(gm.w & 0xffff)), h7 = f2h(v1.w * inv * h2f(gm.w >> 16));
            // groups 2c, 2c + 1 swizzled: (x0, x2), (x1, x3), (x4, x6), (x5, x7)
            u4v d;
            d.x = h0 | (h2 << 16);
            d.y = h1 | (h3 << 16);
            d.z = h4 | (h6 << 16);
            d.w = h5 | (h7 << 16);
            *reinterpret_cast<u4v*>(ar.xs + 4 * c) = d;
            ar.xsum[c] = ((h2f(h0) + h2f(h2)) + (h2f(h1) + h2f(h3))) + ((h2f(h4) + h2f(h6)) + (h2f(h5) + h2f(h7)));
        }
    }
    __syncthreads();
    return true;
}

template <int FQ, int FV, int FO, int FGU, int FD, int FH, int UH, int UO, int UF, int RA, int RC, int RD, int RE,
          int RH, int HD>
__global__ __launch_bounds__(kPT, 1) void persist_kernel(PArgs a) {
    extern __shared__ __align__(16) unsigned char psm[];
    const int H = a.H, F = a.F, qd = a.n_q * HD, kvd = a.n_kv * HD;
    // The layer table goes to LDS first: weight pointers read from global
    // memory would be vector loads, and the wait for one (vmcnt, in order)
    // would also wait for every weight prefetch issued before it.
    bx_decode_layer* const lt = reinterpret_cast<bx_decode_layer*>(psm);
    for (int i = tidx(); i < a.L * (int)(sizeof(bx_decode_layer) / 8); i += kPT)
        reinterpret_cast<uint64_t*>(psm)[i] = gptr<uint64_t>(a.layers)[i];
    __syncthreads();
    const Arena ar = make_arena(psm + layer_table_bytes(a.L), H, F, qd);
    const int G = gridDim.x, w = blockIdx.x;
    const int wave = tidx() >> 6, lane = tidx() & 63;
    const int tok = a.scal[0], pos = a.scal[1];
    stamp(a, 0);
    if (a.trace && tidx() == 0) a.trace[(size_t)blockIdx.x * kTraceSlots + 920] = clock64();

    constexpr int hw = head_words(HD);
    // residual rows owned by this WG (rows of Wo and Wd): whole triples
    int hwb, hwe;
    range_of(words3(H), G, w, hwb, hwe);
    const int hb = 3 * hwb, he = min(3 * hwe, H);

    // embedding row -> hv (all) and own rows
    for (int i = tidx(); i < H; i += kPT) ar.hv[i] = h2f(a.embed[(int64_t)tok * H + i]);
    __syncthreads();
    for (int i = tidx(); i < he - hb; i += kPT) ar.own[i] = ar.hv[hb + i];
    __syncthreads();

    // stage A partition: q / k / v segments (per-head triples) spread over WGs
    // (the host balances bytes and keeps each WG to one task round per wave)
    const int g_v = G - a.g_q - a.g_k;
    int seg, segw, segn;
    if (w < a.g_q) { seg = 0; segw = w; segn = a.g_q; }
    else if (w < a.g_q + a.g_k) { seg = 1; segw = w - a.g_q; segn = a.g_k; }
    else { seg = 2; segw = w - a.g_q - a.g_k; segn = g_v; }
    const int seg_rows = seg == 0 ? qd : kvd;
    uint64_t* const seg_out = seg == 0 ? a.qw : (seg == 1 ? a.kw : a.vw);
    int awb, awe;
    range_of(seg_rows / HD * hw, segn, segw, awb, awe);
    const int ab = head_row<HD>(awb), ae = head_row<HD>(awe);
    int fwb, fwe;   // SwiGLU outputs (gate/up rows): whole triples
    range_of(words3(F), G, w, fwb, fwe);
    const int fb = 3 * fwb, fe = min(3 * fwe, F);
    auto head_nrows = [](int W) { return max(0, min(3, HD - 3 * (W % hw))); };
    auto flat_row = [](int W) { return 3 * W; };

    // Weight blocks of each wave's first task per stage, requested ahead of
    // their input: A(l) before its residual poll, C(l) while A(l) computes,
    // D(l) while C(l) computes, E(l) while D(l) computes.  Further tasks (rows
    // beyond one task per wave) load in place.
    const int a0 = ab + wave * RA, c0r = hb + wave * RC, d0 = fb + wave * RD, e0 = hb + wave * RE;

    // A blocks are requested during E of the layer before (the first layer's
    // here), so that they have landed before A's residual poll: loads complete
    // in issue order, and a poll issued behind fresh weight loads waits for them.
    // A workgroup loads the rows of one segment only, so when q / k and v share
    // a format one block serves all three: two blocks live across the layer
    // loop would not fit the registers of the widest shapes.
    RowBlock<FQ, UH, RA> wa_qk;
    std::conditional_t<FQ == FV, char, RowBlock<FV, UH, RA>> wa_v_own;
    RowBlock<FV, UH, RA>& wa_v = [&]() -> RowBlock<FV, UH, RA>& {
        if constexpr (FQ == FV) return wa_qk;
        else return wa_v_own;
    }();
    auto issue_a = [&](const bx_decode_layer& L, int z) {
        if (a0 < ae) {
            if (seg == 2) wa_v.load(L.Wv, kvd, H, a0 + z);
            else wa_qk.load(seg == 0 ? L.Wq : L.Wk, seg_rows, H, a0 + z);
        }
    };
    attn_tile_prefetch<HD>(a, ar, lt[0], pos, opaque_zero());
    issue_a(lt[0], opaque_zero());
    pin_loads<1>();

    for (int l = 0; l < a.L; ++l) {
        const bx_decode_layer& Ly = lt[l];
        const int zl = opaque_zero();
        // declared per layer: a block is live only from its load to its use
        RowBlock<FO, UO, RC> wc;
        RowBlock<FGU, UH, RD> wg, wu;
        RowBlock<FD, UF, RE> we;
        const int sl = 1 + 10 * l;
        // ---- A: norm + q/k/v rows
        {
            GammaRegs gam;
            gam.load(Ly.in_ln, H);
            if (!poll_norm(a, ar, l > 0 ? a.hbuf + zl : nullptr, tag_of(a, l - 1, 4), 1, gam, a.eps)) return;
            stamp(a, sl + 0);
            const uint32_t t = tag_of(a, l, 0);
            auto put = [&](int r, const float(&o)[RA]) {
                if (lane == 0) {
#pragma unroll
                    for (int rr = 0; rr < RA; ++rr)
                        if (r + rr < ae) ar.rows[r + rr - ab] = o[rr];
                }
            };
            if (seg == 2) {
                XCache<FV, UH> xu;
                xu.init(ar.xs, ar.xsum, H);
                peeled_tasks(
                    a0, ae, kPW * RA, [&](int r) { wa_v.load(Ly.Wv, kvd, H, r + zl); },
                    [&](int r) {
                        float o[RA];
                        wa_v.dot(H, xu, o);
                        put(r, o);
                    });
            } else {
                const void* W = seg == 0 ? Ly.Wq : Ly.Wk;
                XCache<FQ, UH> xu;
                xu.init(ar.xs, ar.xsum, H);
                peeled_tasks(
                    a0, ae, kPW * RA, [&](int r) { wa_qk.load(W, seg_rows, H, r + zl); },
                    [&](int r) {
                        float o[RA];
                        wa_qk.dot(H, xu, o);
                        put(r, o);
                    });
            }
            __syncthreads();
            emit_triples(ar.rows, seg_out + zl, awb, awe, ab, t, [](int W) { return head_row<HD>(W); }, head_nrows);
            // C's weights stream while q / k / v travel to the attention splits
            wc.load(Ly.Wo, H, qd, c0r + zl);
            pin_loads<2>();
        }
        __syncthreads();
        stamp(a, sl + 1);
        // ---- B: attention
        if (!__syncthreads_and(attention_stage<HD>(a, ar, Ly, l, pos, zl))) return;
        stamp(a, sl + 2);
        // ---- C: o-proj + residual
        {
            if (!poll_triples_to_xs<2>(a, ar, a.attn + zl, a.n_q * hw, qd, tag_of(a, l, 1), 2,
                                       [](int i, int j) { return head_elem<HD>(i, j); }))
                return;
            stamp(a, sl + 3);
            const uint32_t t = tag_of(a, l, 2);
            {
                XCache<FO, UO> xu;
                xu.init(ar.xs, ar.xsum, qd);
                peeled_tasks(c0r, he, kPW * RC, [&](int r) { wc.load(Ly.Wo, H, qd, r + zl); }, [&](int r) {
                    float o[RC];
                    wc.dot(qd, xu, o);
                    if (lane == 0) {
#pragma unroll
                        for (int rr = 0; rr < RC; ++rr)
                            if (r + rr < he) ar.own[r + rr - hb] += o[rr];
                    }
                });
            }
            __syncthreads();
            emit_triples(ar.own, a.hbuf + zl, hwb, hwe, hb, t, flat_row, [&](int W) { return min(3, H - 3 * W); });
            // D's weights stream while the residual travels to the norm
            wg.load(Ly.Wg, F, H, d0 + zl);
            wu.load(Ly.Wu, F, H, d0 + zl);
            pin_loads<3>();
        }
        __syncthreads();
        stamp(a, sl + 4);
        // ---- D: norm + gate/up row pairs
        {
            GammaRegs gam;
            gam.load(Ly.post_ln, H);
            if (!poll_norm(a, ar, a.hbuf + zl, tag_of(a, l, 2), 3, gam, a.eps)) return;
            stamp(a, sl + 5);
            const uint32_t t = tag_of(a, l, 3);
            {
                XCache<FGU, UH> xu;
                xu.init(ar.xs, ar.xsum, H);
                if (l == kTraceLayer) stamp(a, 910);
                auto load = [&](int r) {
                    wg.load(Ly.Wg, F, H, r + zl);
                    wu.load(Ly.Wu, F, H, r + zl);
                };
                peeled_tasks(d0, fe, kPW * RD, load, [&](int r) {
                    float gg[RD], uu[RD];
                    wg.dot(H, xu, gg);
                    if (l == kTraceLayer) stamp(a, 911);
                    wu.dot(H, xu, uu);
                    if (l == kTraceLayer) stamp(a, 912);
                    if (lane == 0) {
#pragma unroll
                        for (int rr = 0; rr < RD; ++rr)
                            if (r + rr < fe) ar.rows[r + rr - fb] = gg[rr] / (1.0f + __expf(-gg[rr])) * uu[rr];
                    }
                });
            }
            __syncthreads();
            if (l == kTraceLayer) stamp(a, 913);
            emit_triples(ar.rows, a.act + zl, fwb, fwe, fb, t, flat_row, [&](int W) { return min(3, F - 3 * W); });
            // E's weights stream while the SwiGLU output travels to the down-proj
            we.load(Ly.Wd, H, F, e0 + zl);
            pin_loads<4>();
        }
        __syncthreads();
        stamp(a, sl + 6);
        // ---- E: down + residual
        {
            if (!poll_triples_to_xs<4>(a, ar, a.act + zl, words3(F), F, tag_of(a, l, 3), 4,
                                       [&](int i, int j) { return 3 * i + j < F ? 3 * i + j : -1; }))
                return;
            stamp(a, sl + 7);
            const uint32_t t = tag_of(a, l, 4);
            {
                XCache<FD, UF> xu;
                xu.init(ar.xs, ar.xsum, F);
                peeled_tasks(e0, he, kPW * RE, [&](int r) { we.load(Ly.Wd, H, F, r + zl); }, [&](int r) {
                    float o[RE];
                    we.dot(F, xu, o);
                    if (lane == 0) {
#pragma unroll
                        for (int rr = 0; rr < RE; ++rr)
                            if (r + rr < he) ar.own[r + rr - hb] += o[rr];
                    }
                });
            }
            __syncthreads();
            emit_triples(ar.own, a.hbuf + zl, hwb, hwe, hb, t, flat_row, [&](int W) { return min(3, H - 3 * W); });
            // the next layer's A weights and first attention tile stream while
            // the residual travels to its norm
            if (l + 1 < a.L) {
                // the tile first: the compiler waits for every earlier load
                // before an LDS-DMA issue, and the A weights are not needed yet
                attn_tile_prefetch<HD>(a, ar, lt[l + 1], pos, zl);
                issue_a(lt[l + 1], zl);
            }
            pin_loads<5>();
        }
        __syncthreads();
        stamp(a, sl + 8);
    }

    // ---- head: final norm, lm_head rows, per-WG argmax
    const int sh = 1 + 10 * a.L;
    int vb, ve;
    range_of(a.V, G, w, vb, ve);
    float best = -INFINITY;
    int besti = -1;
    {
        // four blocks of RH / 2 rows in turn: three tasks' rows in flight
        static_assert(RH % 2 == 0, "head tasks are RH / 2 rows");
        constexpr int RB = RH / 2;
        RowBlock<FH, UH, RB> hb[4];
        const int first = vb + wave * RB;
        hb[0].load(a.lm_head, a.V, H, first < ve ? first : vb);
        GammaRegs gam;
        gam.load(a.final_norm, H);
        if (!poll_norm(a, ar, a.hbuf, tag_of(a, a.L - 1, 4), 5, gam, a.eps)) return;
        stamp(a, sh + 0);
        head_rows_nb<FH, UH, RB, 4>(hb, a.lm_head, a.V, H, vb, ve, ar, [&](int r, float v) {
            const uint16_t hv16 = f2h(v);
            a.logits[r] = hv16;
            const float q = h2f(hv16);
            if (besti < 0 || q > best) { best = q; besti = r; }
        });
    }
    stamp(a, sh + 1);
    if (a.trace && tidx() == 0) {
        a.trace[(size_t)blockIdx.x * kTraceSlots + 921] = clock64();
        a.trace[(size_t)blockIdx.x * kTraceSlots + 922] = wall_clock64();
    }
    // WG argmax: lane 0 of each wave holds its best (lowest index among equal values).
    float* rv = ar.red;
    int* ri = reinterpret_cast<int*>(ar.red + 8);
    __syncthreads();
    if (lane == 0) {
        rv[wave] = best;
        ri[wave] = besti;
    }
    __syncthreads();
    const uint32_t tc = tag_of(a, a.L, 0);
    if (tidx() == 0) {
        float bv = -INFINITY;
        int bi = -1;
        for (int i = 0; i < kPW; ++i) {
            if (ri[i] < 0) continue;
            if (bi < 0 || rv[i] > bv || (rv[i] == bv && ri[i] < bi)) { bv = rv[i]; bi = ri[i]; }
        }
        st_u32(a.cand + 2 * w, tc, __float_as_uint(bv));
        st_u32(a.cand + 2 * w + 1, tc, (uint32_t)bi);
    }
    if (w != 0) return;
    float* cv = ar.att;  // 2G values
    const bool ok = poll_words<1>(a, a.cand, 2 * G, tc, 6, [&](int i, uint64_t v) { cv[i] = __uint_as_float(word_lo(v)); });
    if (!__syncthreads_and(ok)) return;
    if (wave == 0) {
        // lanes scan strided candidates, then a shuffle tree keeps (max value, lowest index)
        float bv = -INFINITY;
        int bi = -1;
        for (int i = lane; i < G; i += 64) {
            const int idx = (int)__float_as_uint(cv[2 * i + 1]);
            const float v = cv[2 * i];
            if (idx < 0) continue;
            if (bi < 0 || v > bv || (v == bv && idx < bi)) { bv = v; bi = idx; }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (lane != 0) return;
        int32_t* scal = a.scal;
        scal[2] = bi;
        scal[0] = bi;
        scal[1] = pos + 1;
        const int32_t c = scal[3];
        scal[4 + c] = bi;
        scal[3] = c + 1;
    }
    stamp(a, sh + 2);
}

struct PKey {
    int fq, fv, fo, fgu, fd, fh, uh, uo, uf, hd;
};

using PFn = void (*)(PArgs);

#define BX_PK(FQ, FV, FO, FGU, FD, FH, UH, UO, UF, RA, RC, RD, RE, RH, HD)           \
    {{FQ, FV, FO, FGU, FD, FH, UH, UO, UF, HD},                                      \
     persist_kernel<FQ, FV, FO, FGU, FD, FH, UH, UO, UF, RA, RC, RD, RE, RH, HD>, RA, RC, RD, RE}

struct PEntry {
    PKey k;
    PFn fn;
    int ra, rc, rd, re;
};

// Instantiated shapes: the common quantization mixes at their widths and the
// small test models of the same mixes.  RA..RH: rows per wave task of stages
// A, C, D (per matrix), E and the head.  Rows per workgroup come in whole
// triples of the hand-off words; RC / RE cover ceil(words3(H) / CUs) triples in
// one round of the four waves where the blocks fit the registers, and in
// several rounds of smaller tasks where they do not.
const PEntry kPersistTable[] = {
    // Q4_K with Q6_K v/down/output (1.7B: H 2048, F 6144; test: H 256, F 768)
    BX_PK(FMT_Q4_K, FMT_Q6_K, FMT_Q4_K, FMT_Q4_K, FMT_Q6_K, FMT_Q6_K, 1, 1, 3, 5, 3, 6, 3, 8, 128),
    BX_PK(FMT_Q4_K, FMT_Q6_K, FMT_Q4_K, FMT_Q4_K, FMT_Q6_K, FMT_Q6_K, 1, 1, 1, 5, 3, 6, 3, 8, 64),
    // all Q8_0, tied FP16 lm_head (0.6B: H 1024, F 3072, qd 2048; test: H 512, F 1024, qd 512)
    BX_PK(FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_F16, 1, 1, 2, 4, 2, 6, 2, 4, 128),
    BX_PK(FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_Q8_0, FMT_F16, 1, 1, 1, 4, 2, 6, 2, 4, 64),
    // Q4_K everywhere with Q6_K output (8B: H 4096, F 12288); A and E in tasks
    // of 2 rows: larger blocks held across the stage boundaries spill registers
    // to scratch at these widths (measured 250 tok/s at RA 6 / RE 5 against
    // 389 tok/s here)
    BX_PK(FMT_Q4_K, FMT_Q4_K, FMT_Q4_K, FMT_Q4_K, FMT_Q4_K, FMT_Q6_K, 2, 2, 6, 2, 5, 4, 2, 4, 128),
    // Q4_K with Q6_K v/down/output at Llama-3-8B widths (H 4096, F 14336, no
    // QK-norm): 1-row A and E tasks keep the Q6_K E blocks (7 units a lane) and
    // the two A blocks in registers (397 tok/s against 368 for the graph step)
    BX_PK(FMT_Q4_K, FMT_Q6_K, FMT_Q4_K, FMT_Q4_K, FMT_Q6_K, FMT_Q6_K, 2, 2, 7, 1, 3, 3, 1, 4, 128),
};

struct PLayout {
    size_t ctrl, hbuf, qw, kw, vw, attn, act, part, cand, total;
    size_t part_stride;   // words per KV group
    size_t lds;
    int smax;
    int g_q, g_k;         // stage A workgroups of the q and k segments (v: the rest)
    PFn fn;
};

// Stage A split of the per-head q / k / v triples over G workgroups: every
// segment gets at least the workgroups that keep each one within one task
// round of its waves (cap words), spare workgroups go one by one to the
// segment with the most bytes per workgroup.  Without room for one round,
// proportional to bytes.
static void split_stage_a(int G, const int (&words)[3], const double (&bpw)[3], int cap, int (&n)[3]) {
    int sum = 0;
    for (int i = 0; i < 3; ++i) {
        n[i] = (words[i] + cap - 1) / cap;
        sum += n[i];
    }
    if (sum > G) {
        const double tot = words[0] * bpw[0] + words[1] * bpw[1] + words[2] * bpw[2];
        sum = 0;
        for (int i = 0; i < 3; ++i) {
            n[i] = (int)(G * words[i] * bpw[i] / tot);
            if (n[i] < 1) n[i] = 1;
            sum += n[i];
        }
        while (sum > G) {
            const int i = n[0] >= n[1] && n[0] >= n[2] ? 0 : (n[1] >= n[2] ? 1 : 2);
            --n[i];
            --sum;
        }
    }
    while (sum < G) {
        int best = 0;
        double bb = -1.0;
        for (int i = 0; i < 3; ++i) {
            const double per = words[i] * bpw[i] / n[i];
            if (per > bb) { bb = per; best = i; }
        }
        ++n[best];
        ++sum;
    }
}

int persist_layout(const bx_decode_dims& d, int G, PLayout& o) {
    const int hd = d.head_dim, qd = d.n_q * hd;
    if (d.n_kv <= 0 || d.n_q % d.n_kv) return fail(BX_EINVAL, "persist: bad head counts");
    const int Gq = d.n_q / d.n_kv;
    if (Gq > kMaxGq) return fail(BX_EUNSUPPORTED, "persist: more than 8 query heads per KV head");
    if (hd != 64 && hd != 128) return fail(BX_EUNSUPPORTED, "persist: head_dim must be 64 or 128");
    if (Gq * hd > kPT * 4) return fail(BX_EUNSUPPORTED, "persist: too many query heads per KV head for head_dim");
    if (d.hidden > 4 * 4 * kPT) return fail(BX_EUNSUPPORTED, "persist: hidden above 4096");
    if (d.qkv_type_q != d.qkv_type_k || d.gate_type != d.up_type)
        return fail(BX_EUNSUPPORTED, "persist: q/k or gate/up formats differ");
    // one format per role across layers (the step is instantiated per format
    // mix); a file that mixes attn_v / ffn_down types by layer runs the
    // per-stage step, which reads each layer's types
    if ((d.v_alt_type && d.v_alt_type != d.qkv_type_v) || (d.down_alt_type && d.down_alt_type != d.down_type))
        return fail(BX_EUNSUPPORTED, "persist: per-layer attn_v / ffn_down types differ");
    if (d.hidden % 256 || d.intermediate % 256 || qd % 256) return fail(BX_EUNSUPPORTED, "persist: widths");
    const int smax = G / d.n_kv;
    if (smax < 1 || G < 3) return fail(BX_EUNSUPPORTED, "persist: too few CUs");
    // every attention split holds its keys in one LDS tile
    if ((int64_t)d.cap > (int64_t)smax * kTile) return fail(BX_EUNSUPPORTED, "persist: KV cache longer than the splits' tiles");
    // a combiner's lanes hold at most two partials each (S P <= 128)
    if ((int64_t)std::min(smax, (d.cap + kSplitQ - 1) / kSplitQ) * att_parts(Gq) > 128)
        return fail(BX_EUNSUPPORTED, "persist: more than 128 attention partials per head");
    const PKey want{d.qkv_type_q, d.qkv_type_v, d.o_type, d.gate_type, d.down_type, d.lm_type,
                    upl_for(d.hidden), upl_for(qd), upl_for(d.intermediate), hd};
    const PEntry* ent = nullptr;
    for (const PEntry& e : kPersistTable) {
        if (e.k.fq == want.fq && e.k.fv == want.fv && e.k.fo == want.fo && e.k.fgu == want.fgu &&
            e.k.fd == want.fd && e.k.fh == want.fh && e.k.uh == want.uh && e.k.uo == want.uo && e.k.uf == want.uf &&
            e.k.hd == want.hd)
            ent = &e;
    }
    if (!ent) return fail(BX_EUNSUPPORTED, "persist: no instantiation for this format mix / width");
    o.fn = ent->fn;
    // rows per workgroup of the residual and SwiGLU triples (LDS holds kMaxOwn)
    const int hw = head_words(hd);
    if (3 * ((words3(d.hidden) + G - 1) / G) > kMaxOwn || 3 * ((words3(d.intermediate) + G - 1) / G) > kMaxOwn)
        return fail(BX_EUNSUPPORTED, "persist: hidden / intermediate too wide for the grid");
    // stage A split
    auto row_bytes = [&](int t) {
        return (double)type_block_bytes(t) * (double)(d.hidden / type_block_elems(t));
    };
    const int words[3] = {d.n_q * hw, d.n_kv * hw, d.n_kv * hw};
    const double bpw[3] = {3 * row_bytes(d.qkv_type_q), 3 * row_bytes(d.qkv_type_k), 3 * row_bytes(d.qkv_type_v)};
    int n[3];
    split_stage_a(G, words, bpw, kPW * ent->ra / 3, n);
    for (int i = 0; i < 3; ++i)
        if (n[i] < 1 || 3 * ((words[i] + n[i] - 1) / n[i]) > kMaxOwn)
            return fail(BX_EUNSUPPORTED, "persist: q / k / v too wide for the grid");
    o.g_q = n[0];
    o.g_k = n[1];
    // LDS: the arena, with the attention scratch grown to a combiner's records
    // or the head's 2G argmax candidates if either is larger
    const size_t att_bytes = att_scratch_bytes(hd, Gq);
    const size_t comb_bytes = comb_lds_floats(hd, Gq, smax) * 4;
    size_t lds = arena_bytes(d.hidden, d.intermediate, qd, hd, Gq);
    if (comb_bytes > att_bytes) lds += comb_bytes - att_bytes;
    if ((size_t)2 * G * 4 > att_bytes) return fail(BX_EUNSUPPORTED, "persist: candidate buffer");
    if (lds > 160 * 1024) return fail(BX_EUNSUPPORTED, "persist: LDS budget exceeded");
    size_t off = 0;
    auto take = [&](size_t words_) {
        const size_t r = off;
        off += (words_ * 8 + 255) / 256 * 256;
        return r;
    };
    o.ctrl = take(32);
    o.hbuf = take(words3(d.hidden));
    o.qw = take((size_t)d.n_q * hw);
    o.kw = take((size_t)d.n_kv * hw);
    o.vw = take((size_t)d.n_kv * hw);
    o.attn = take((size_t)d.n_q * hw);
    o.act = take(words3(d.intermediate));
    o.part_stride = (part_words_per_group(hd, Gq, smax) + 1) & ~(size_t)1;
    o.part = take((size_t)d.n_kv * o.part_stride);
    o.cand = take((size_t)2 * G);
    o.total = off;
    o.lds = lds;
    o.smax = smax;
    return BX_OK;
}

int persist_grid() { return num_cus(); }

uint64_t* g_trace = nullptr;   // set by bx_persist_trace

// Workspace (re)initialization: control block zeroed (no abort), every
// hand-off word all-ones (a tag no step writes).
__global__ void persist_ws_init_kernel(uint32_t* ctrl, uint64_t* words, size_t nwords) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 64) ctrl[i] = 0u;
    for (size_t j = i; j < nwords; j += (size_t)gridDim.x * blockDim.x) words[j] = ~0ull;
}

}  // namespace

// The first persistent step, kept for the shapes persist2.hip has no
// instantiation for; the bx_persist_* entry points (persist2.hip) call these.
size_t p1_ws_bytes(const bx_decode_dims* d) {
    if (!d) return 0;
    bx::PLayout o{};
    if (bx::persist_layout(*d, bx::persist_grid(), o) != BX_OK) return 0;
    return o.total;
}

int p1_ws_init(const bx_decode_dims* d, void* ws, void* stream) {
    if (!d || !ws) return bx::fail(BX_EINVAL, "persist_ws_init: null pointer");
    bx::PLayout o{};
    if (int rc = bx::persist_layout(*d, bx::persist_grid(), o)) return rc;
    unsigned char* base = static_cast<unsigned char*>(ws);
    const size_t nwords = (o.total - o.hbuf) / 8;
    hipLaunchKernelGGL(bx::persist_ws_init_kernel, dim3(256), dim3(256), 0, bx::as_stream(stream),
                       reinterpret_cast<uint32_t*>(base + o.ctrl), reinterpret_cast<uint64_t*>(base + o.hbuf), nwords);
    if (hipGetLastError() != hipSuccess) return bx::fail(BX_ELAUNCH, "persist_ws_init: launch failed");
    return BX_OK;
}

int p1_step(const bx_decode_dims* d, int n_layers, const bx_decode_layer* layers_dev, const uint16_t* embed,
            const uint16_t* final_norm, const void* lm_head, const float* cos_tab, const float* sin_tab, int32_t* scal,
            uint16_t* logits, void* ws, uint32_t epoch, void* stream) {
    if (!d || !layers_dev || !embed || !final_norm || !lm_head || !cos_tab || !sin_tab || !scal || !logits || !ws)
        return bx::fail(BX_EINVAL, "persist: null pointer");
    if (n_layers <= 0 || n_layers > 126) return bx::fail(BX_EINVAL, "persist: layer count");
    if (epoch == 0 || epoch >= 64) return bx::fail(BX_EINVAL, "persist: epoch out of range (1..63)");
    const int G = bx::persist_grid();
    bx::PLayout o{};
    if (int rc = bx::persist_layout(*d, G, o)) return rc;
    const int hd = d->head_dim;
    bx::PArgs a{};
    a.H = d->hidden; a.F = d->intermediate; a.n_q = d->n_q; a.n_kv = d->n_kv; a.hd = hd; a.V = d->vocab;
    a.cap = d->cap; a.L = n_layers; a.eps = d->eps; a.qk_norm = d->no_qk_norm ? 0 : 1;
    a.g_q = o.g_q; a.g_k = o.g_k;
    a.epoch = epoch;
    a.layers = layers_dev;
    a.embed = embed; a.final_norm = final_norm; a.lm_head = lm_head; a.cos_t = cos_tab; a.sin_t = sin_tab;
    a.scal = scal; a.logits = logits;
    unsigned char* base = static_cast<unsigned char*>(ws);
    a.ctrl = reinterpret_cast<uint32_t*>(base + o.ctrl);
    a.hbuf = reinterpret_cast<uint64_t*>(base + o.hbuf);
    a.qw = reinterpret_cast<uint64_t*>(base + o.qw);
    a.kw = reinterpret_cast<uint64_t*>(base + o.kw);
    a.vw = reinterpret_cast<uint64_t*>(base + o.vw);
    a.attn = reinterpret_cast<uint64_t*>(base + o.attn);
    a.act = reinterpret_cast<uint64_t*>(base + o.act);
    a.part = reinterpret_cast<uint64_t*>(base + o.part);
    a.part_stride = (int64_t)o.part_stride;
    a.cand = reinterpret_cast<uint64_t*>(base + o.cand);
    a.trace = bx::g_trace;
    hipStream_t st = bx::as_stream(stream);
    o.lds += bx::layer_table_bytes(n_layers);
    if (o.lds > 160 * 1024) return bx::fail(BX_EUNSUPPORTED, "persist: LDS budget exceeded (layer table)");
    if (o.lds > 64 * 1024) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(o.fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)o.lds) != hipSuccess)
            return bx::fail(BX_ELAUNCH, "persist: cannot raise the LDS limit");
    }
    void* args[] = {&a};
    // A plain launch of the grid after the occupancy check the cooperative
    // launch makes (one workgroup per CU, grid = CU count), so the grid is
    // co-resident on a device no other kernel holds, without the cooperative
    // launch's cost (about 18 us a step).  Every wait is bounded and raises
    // the abort flag, so the kernel ends either way.  BROLM_PERSIST_COOPERATIVE=1
    // takes the cooperative launch, except under a profiler tool (rocprofv3
    // has ended processes whose kernels were launched cooperatively with a
    // segmentation fault in its exit path).
    static const bool plain = std::getenv("BROLM_PERSIST_COOPERATIVE") == nullptr || bx::profiler_attached();
    hipError_t e;
    if (plain) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(o.fn), bx::kPT,
                                                          o.lds) != hipSuccess ||
            per_cu < 1)
            return bx::fail(BX_ELAUNCH, "persist: workgroup does not fit on a CU");
        e = hipLaunchKernel(reinterpret_cast<const void*>(o.fn), dim3(G), dim3(bx::kPT), args, o.lds, st);
    } else {
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(o.fn), dim3(G), dim3(bx::kPT), args,
                                       (unsigned)o.lds, st);
    }
    if (e != hipSuccess) return bx::fail(BX_ELAUNCH, std::string("persist: launch failed: ") + hipGetErrorString(e));
    return BX_OK;
}

void p1_set_trace(uint64_t* buf) { g_trace = buf; }

}  // namespace bx
