// Persistent single-launch decode step, partitioned by XCD.
//
// The L = 1 step of src/detail/dense_decoder.cpp:439-496 (run_layers_,
// :526-681, at one token): embedding, every layer, final norm, lm_head,
// greedy argmax and the token feedback, as ONE launch of 256 co-resident
// workgroups, one per CU: 32 on each of the 8 XCDs, each XCD with its own L2.
// The dispatcher deals workgroups to the XCDs in turn, starting wherever the
// previous launch left off, so a workgroup reads its XCD from HW_REG_XCC_ID
// and takes a rank among the XCD's workgroups from a counter in that L2; the
// kernel works on these (XCD, rank) ids, never on blockIdx.  Hand-offs inside
// an XCD go through its L2 (plain stores, sc0|nt loads); hand-offs between
// XCDs go through memory (sc1 stores and loads) and cost about twice as
// much.  The work is split so that a layer needs two cross-XCD hand-offs:
//
//   XCD x owns attention unit x (gpu consecutive KV groups: their q / k / v
//   rows, their attention and the Wo columns that read their heads) and FFN
//   slice x (gate / up rows and the Wd columns of a contiguous F range).
//   Wo and Wd then produce per-XCD partial sums of the residual update.
//
//   Every workgroup keeps the whole residual h (FP32) in its LDS and adds the
//   XCDs' partials to it in XCD order, so every copy holds the same bits and
//   no workgroup has to broadcast h.
//
// Per layer, workgroup r (0..31) of XCD x:
//   A  [cross] down partials of layer l-1 -> h; RMSNorm -> rows of the unit's
//      Wq / Wk / Wv (segments spread over the 32 workgroups)  -> local words
//   B  [local] q / k / v of the unit -> (group, key split) = (r mod gpu,
//      r / gpu): QK-norm, RoPE, KV row, scores, softmax, P.V over the split's
//      keys (an LDS tile prefetched one layer ahead) -> a normalized partial
//      record per head                                         -> local words
//   C  [local] the records -> attention output of the unit's heads (FP16) ->
//      H / 32 rows of Wo over the unit's columns              -> cross words
//   D  [cross] Wo partials -> h; RMSNorm -> gate / up rows of slice x ->
//      silu(g) u                                               -> local words
//   E  [local] slice x of the SwiGLU output -> H / 32 rows of Wd over the
//      slice's columns                                          -> cross words
// Head: [cross] down partials -> h; RMSNorm -> V / 256 lm_head rows, per-WG
// argmax; workgroup 0 reduces the candidates and advances tok / pos.
//
// A hand-off word is 64 bits: a 16-bit tag (epoch mod 64, layer, stage) and
// three FP16 values or one 32-bit value.  Every wait polls words until their
// tags match, is bounded, and raises a shared abort flag when it gives up, so
// every wave leaves the kernel whatever happens.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>

#include "gemv_core.h"

namespace bx {

// the first persistent kernel (persist.hip), the fallback for shapes this one
// does not cover
size_t p1_ws_bytes(const bx_decode_dims* d);
int p1_ws_init(const bx_decode_dims* d, void* ws, void* stream);
int p1_step(const bx_decode_dims* d, int n_layers, const bx_decode_layer* layers_dev, const uint16_t* embed,
            const uint16_t* final_norm, const void* lm_head, const float* cos_tab, const float* sin_tab,
            int32_t* scal, uint16_t* logits, void* ws, uint32_t epoch, void* stream);
void p1_set_trace(uint64_t* buf);

namespace p2 {
namespace {

// Per-shape code options (the OPT template argument of the kernel, chosen by
// measurement per table entry):
//   kLate    a stage requests the next stage's weights after emitting its own
//            output words instead of before its dot products;
//   kAsmDma  the attention tile's LDS-DMA copies are issued from inline
//            assembly.  The compiler's wait-count pass does not see them, so it
//            stops making every later LDS read wait for every outstanding
//            global load (it cannot tell the tile's DMA writes from other LDS
//            data); the copies are waited for explicitly (s_waitcnt 0) before
//            the barrier that publishes the tile.
constexpr int kLate = 1, kAsmDma = 2;

constexpr int kT = 256;          // threads per workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kX = 8;            // XCDs
constexpr int kR = 32;           // workgroups per XCD
constexpr int kG = kX * kR;      // grid
constexpr int kTile = 128;       // keys per attention split at most (one LDS tile)
constexpr int kMinKeys = 64;     // keys per split before a further split opens
constexpr int kMaxGq = 8;
constexpr uint32_t kSpinCheck = 128;        // poll rounds between abort checks
constexpr uint32_t kSpinLimit = 1u << 21;   // poll rounds before giving up
constexpr int kTraceSlots = 1024;
constexpr uint32_t kSiteXcd = 99;           // abort site: more than 32 workgroups on one XCD
constexpr int kCtrlWords = 64;              // ctrl[0] abort flag, [1] site; then the rank counters
constexpr int kCtrlBytes = 4 * (kCtrlWords + 64 * kX);

// Load cache policies of the polls (buffer-load aux bits): sc0|nt reads an
// XCD-local word from the L2 without keeping a stale copy in the CU's L1;
// sc1 reads through to memory, where sc1 stores of other XCDs land.
constexpr int kLocal = 3;
constexpr int kCross = 16;

struct Args {
    int H, F, nq, nkv, V, cap, L;
    float eps;
    int qk_norm;
    uint32_t epoch;
    // plan (host-computed)
    int gpu, nu;            // KV groups per attention unit; units (= XCDs 0 .. nu-1 with attention)
    int aq, ak, av;         // stage A workgroups of the q, k and v segments (aq + ak + av = 32)
    int wq, wk, wv;         // hand-off words per workgroup of each segment (even)
    int wqkv;               // words of a unit's q / k / v vector
    int smax;               // key splits per group at most (32 / gpu)
    int rec;                // words per attention record (even)
    int fblk;               // FFN slice granularity (elements)
    int wact;               // SwiGLU words per workgroup (even)
    int wpart;              // h-update words per workgroup (even), ceil(H / 32 / 3) rounded up
    const bx_decode_layer* layers;
    const uint16_t* embed;
    const uint16_t* final_norm;
    const void* lm_head;
    const float* cos_t;
    const float* sin_t;
    int32_t* scal;          // tok, pos, next, count, hist[...]
    uint16_t* logits;
    uint32_t* ctrl;         // [0] abort flag, [1] site, [kCtrlWords + 8 epoch + x] rank counters
    uint64_t* qkv;          // local, [kX][qkv_stride]
    uint64_t* recw;         // local, [kX][rec_stride]
    uint64_t* act;          // local, [kX][act_stride]
    uint64_t* pwo;          // cross, [kX][part_stride]: Wo partials, one FP32 row per word
    uint64_t* pdn;          // cross, [kX][part_stride]: Wd partials
    uint64_t* hupo;         // local, [kX][hup_stride]: summed Wo update of h (FP16 triples)
    uint64_t* hupd;         // local, [kX][hup_stride]: summed Wd update of h
    uint64_t* cand;         // cross, [2 kG]
    int qkv_stride, rec_stride, act_stride, part_stride, hup_stride;
    uint64_t* trace;
};

// ---- tagged words ------------------------------------------------------------

__host__ __device__ constexpr int words3(int n) { return (n + 2) / 3; }
__host__ __device__ constexpr int even(int n) { return (n + 1) & ~1; }

__device__ __forceinline__ uint32_t tag_of(const Args& a, int layer, int stage) {
    return ((a.epoch & 63u) << 10) | ((uint32_t)layer << 3) | (uint32_t)stage;
}
__device__ __forceinline__ uint64_t word3(uint32_t tag, uint32_t v0, uint32_t v1, uint32_t v2) {
    return ((uint64_t)tag << 48) | ((uint64_t)v2 << 32) | ((uint64_t)v1 << 16) | (uint64_t)v0;
}
__device__ __forceinline__ uint64_t word1(uint32_t tag, uint32_t v) { return ((uint64_t)tag << 48) | v; }
// XCD-local hand-off: a plain store, which lands in the XCD's L2.
__device__ __forceinline__ void st_local(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Cross-XCD hand-off: a device-scope store (sc1), written through to memory.
__device__ __forceinline__ void st_cross(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fld(uint32_t lo, uint32_t hi, int j) {
    return j == 0 ? (lo & 0xffffu) : (j == 1 ? (lo >> 16) : (hi & 0xffffu));
}

// The thread index through an opaque move, so per-lane addresses derived
// from it are not hoisted out of the layer loop (where dozens of them would
// outlive the register file).
__device__ __forceinline__ int tidx() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return z;
}
// Compiler barrier: loads issued before it stay before it (prefetches are
// not sunk to their first use).
__device__ __forceinline__ void pin() { asm volatile("" ::: "memory"); }

// x / d for 0 <= x < 2^16 and 1 <= d <= 2^16 by a multiply-high with
// ceil(2^32 / d): the error x / 2^32 < 2^-16 never crosses an integer, since
// the fractional parts of x / d are multiples of 1 / d.
struct FastDivP {
    uint32_t d, m;
    __device__ __forceinline__ explicit FastDivP(int d_)
        : d((uint32_t)d_), m((uint32_t)(0xffffffffu / (uint32_t)d_) + 1u) {}
    __device__ __forceinline__ int div(int x) const { return d == 1 ? x : (int)__umulhi((uint32_t)x, m); }
};

__device__ __forceinline__ void stamp(const Args& a, int slot) {
    if (a.trace && tidx() == 0) a.trace[(size_t)blockIdx.x * kTraceSlots + slot] = wall_clock64();
}

// Sub-stage stamps of layer 14 (slots 600 + k).
__device__ __forceinline__ void sub(const Args& a, int l, int k) {
    if (l == 14) stamp(a, 600 + k);
}

__device__ __forceinline__ bool aborted(const Args& a) {
    return __hip_atomic_load(a.ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void raise_abort(const Args& a, uint32_t site) {
    __hip_atomic_store(a.ctrl + 1, site, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.ctrl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool spin(const Args& a, uint32_t& rounds, uint32_t site) {
    ++rounds;
    if (rounds % kSpinCheck == 0) {
        if (aborted(a)) return false;
        if (rounds >= kSpinLimit) {
            raise_abort(a, site);
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint64_t* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(p), 0, 0x7fffffff, 0x00020000);
}

// Poll word pairs: slot e (< n) is the 16-byte pair at byte offset off[e] of
// rs; returns once both tags of every slot equal `tag` (v holds the pairs),
// false on abort.
template <int E, int AUX>
__device__ __forceinline__ bool poll_slots(const Args& a, __amdgpu_buffer_rsrc_t rs, const int (&off)[E], int n,
                                           uint32_t tag, uint32_t site, u4v (&v)[E]) {
    uint32_t pend = 0;
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (e < n) pend |= 1u << e;
    uint32_t rounds = 0;
    while (pend) {
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (pend & (1u << e)) v[e] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[e], 0, AUX);
#pragma unroll
        for (int e = 0; e < E; ++e)
            if ((pend & (1u << e)) && (v[e][1] >> 16) == tag && (v[e][3] >> 16) == tag) pend &= ~(1u << e);
        if (pend && !spin(a, rounds, site)) return false;
    }
    return true;
}

// Poll the nw (even) words of a contiguous vector, E pairs per thread per
// round; sink(i, lo, hi) for every word i (lo / hi: its two 32-bit halves).
template <int E, int AUX, class Sink>
__device__ __forceinline__ bool poll_vec(const Args& a, const uint64_t* buf, int nw, uint32_t tag, uint32_t site,
                                         Sink sink) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(buf);
    const int np = nw / 2;
    for (int base = 0; base < np; base += E * kT) {
        int off[E];
        int n = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int p = base + tidx() + e * kT;
            off[e] = 16 * (p < np ? p : 0);
            if (p < np) n = e + 1;
        }
        u4v v[E];
        if (!poll_slots<E, AUX>(a, rs, off, n, tag, site, v)) return false;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (e < n) {
                const int p = base + tidx() + e * kT;
                sink(2 * p, v[e][0], v[e][1]);
                sink(2 * p + 1, v[e][2], v[e][3]);
            }
        }
    }
    return true;
}

// ---- reductions over lane groups ------------------------------------------------

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF,
                                                                 false));
}
// Sums of lane groups of LPR (1..64, a power of two) for NP values at once;
// the sum of group g ends in lane sum_lane<LPR>(g).
template <int LPR, int NP>
__device__ __forceinline__ void group_sum(float (&v)[NP]) {
    if constexpr (LPR >= 2)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0xB1>(v[p]);
    if constexpr (LPR >= 4)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0x4E>(v[p]);
    if constexpr (LPR >= 8)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0x141>(v[p]);
    if constexpr (LPR >= 16)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0x140>(v[p]);
    if constexpr (LPR >= 32)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0x142, 0xA>(v[p]);
    if constexpr (LPR >= 64)
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] += dpp<0x143, 0xC>(v[p]);
}
template <int LPR>
__device__ __forceinline__ constexpr int sum_lane(int g) {
    return LPR <= 16 ? g * LPR : g * LPR + LPR - 1;
}

// ---- weight rows ---------------------------------------------------------------

// One 32-element unit of any quant format in registers (48 bytes):
//   Q4_K: a = qs, b = d / dmin / scales;  Q6_K: a = ql, b = scales,
//   c.xy = qh, c.z = d;  Q8_0: a, b = qs, c.x = d.
struct RawAny {
    u4v a, b, c;
};

// A Q4_K or Q6_K unit into RawAny with the same four loads whichever the
// format (`q6` picks the addresses).  A stage whose format is known only at
// run time (attn_v, ffn_down) then requests its rows without a branch: with a
// branch per format the loaded registers meet at the join, and the wave waits
// there for its loads.  Q4_K's last two loads re-read bytes of its own unit.
__device__ __forceinline__ void load_any_kq(RawAny& r, bool q6, const void* W, int64_t N, int64_t K, int64_t n,
                                            int u) {
    const uint8_t* p = static_cast<const uint8_t*>(W);
    const int64_t nb = K / 256, s = n * nb + (u >> 3), plane = N * nb;
    const uint8_t* pa = p + s * 128 + 16 * (u & 7);                        // qs / ql
    const uint8_t* pb = p + plane * (q6 ? 192 : 128) + s * 16;             // header / scales
    const uint8_t* pc = q6 ? p + plane * 128 + s * 64 + 8 * (u & 7) : pa;  // qh
    const uint8_t* pd = q6 ? p + plane * 208 + s * 2 : pb;                 // d
    r.a = ldg_nt16(pa);
    r.b = ldg16(pb);
    const u2v c = ldg_nt8(pc);
    r.c.x = c.x;
    r.c.y = c.y;
    r.c.z = ldg_u16(pd);
}

template <int FMT>
__device__ __forceinline__ void load_any(RawAny& r, const void* W, int64_t N, int64_t K, int64_t n, int u) {
    if constexpr (FMT == FMT_Q4_K) {
        const RawQ4K q = load_unit<FMT_Q4_K>(W, N, K, n, u);
        r.a = q.q;
        r.b = q.h;
    } else if constexpr (FMT == FMT_Q6_K) {
        const RawQ6K q = load_unit<FMT_Q6_K>(W, N, K, n, u);
        r.a = q.ql;
        r.b = q.sc;
        r.c.x = q.qh.x;
        r.c.y = q.qh.y;
        r.c.z = q.d;
    } else if constexpr (FMT == FMT_Q8_0) {
        const RawQ8 q = load_unit<FMT_Q8_0>(W, N, K, n, u);
        r.a = q.q0;
        r.b = q.q1;
        r.c.x = q.d;
    }
}
template <int FMT>
__device__ __forceinline__ float dot_any(const RawAny& r, int u, const XU& x) {
    if constexpr (FMT == FMT_Q4_K) {
        RawQ4K q;
        q.q = r.a;
        q.h = r.b;
        return dot_reg(q, u, x);
    } else if constexpr (FMT == FMT_Q6_K) {
        RawQ6K q;
        q.ql = r.a;
        q.sc = r.b;
        q.qh.x = r.c.x;
        q.qh.y = r.c.y;
        q.d = r.c.z;
        return dot_reg(q, u, x);
    } else {
        RawQ8 q;
        q.q0 = r.a;
        q.q1 = r.b;
        q.d = r.c.x;
        return dot_reg(q, u, x);
    }
}

// The activation units of a lane: unit i of a row is slot + LPR i (slot =
// lane mod LPR), U units per row; units past U repeat unit U - 1 (their
// products are dropped).
template <int FMT, int LPR, int UPL>
struct XRegs {
    XU x[UPL];
    __device__ __forceinline__ void load(const uint32_t* xs, const float* xsum8, int U) {
        const int slot = tidx() & (LPR - 1);
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = slot + LPR * i;
            x[i] = load_xu<FMT>(xs, xsum8, u < U ? u : U - 1);
        }
        pin();
    }
};

// Register storage of one unit: the format's own raw type when a stage has
// one format, RawAny when layers may differ (attn_v / ffn_down).
template <int F1, int F2>
using RawFor = std::conditional_t<(F2 < 0 || F2 == F1), typename RawOf<F1>::T, RawAny>;

// A wave's task: NP passes of 64 / LPR rows (row r0 + p (64 / LPR) + lane /
// LPR), each row by LPR lanes holding UPL units each, over the K-slice of U
// units starting at unit uc0 of the matrix.  Loads are issued unconditionally
// (rows and units clamped into the matrix), so the compiler counts them
// exactly and a task's wait covers only its own loads.
template <class Raw, int LPR, int UPL, int NP>
struct Task {
    static constexpr int RPP = 64 / LPR;   // rows per pass
    Raw raw[NP][UPL];

    // Pass p's units (rows r0 + p (64 / LPR) + lane / LPR, clamped).
    template <int FMT>
    __device__ __forceinline__ void load_pass(const void* W, int64_t N, int64_t K, int uc0, int U, int r0, int p) {
        const int lane = tidx() & 63;
        const int slot = lane & (LPR - 1), rip = lane / LPR;
        int64_t row = r0 + p * RPP + rip;
        row = row < N ? row : N - 1;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = slot + LPR * i;
            const int uu = uc0 + (u < U ? u : U - 1);
            if constexpr (std::is_same_v<Raw, RawAny>) load_any<FMT>(raw[p][i], W, N, K, row, uu);
            else raw[p][i] = load_unit<FMT>(W, N, K, row, uu);
        }
    }
    template <int FMT>
    __device__ __forceinline__ void load(const void* W, int64_t N, int64_t K, int uc0, int U, int r0) {
#pragma unroll
        for (int p = 0; p < NP; ++p) load_pass<FMT>(W, N, K, uc0, U, r0, p);
    }
    // Pass p of a Q4_K or Q6_K matrix whose format is a run-time value
    // (RawAny storage only): the same loads either way.
    __device__ __forceinline__ void load_pass_kq(bool q6, const void* W, int64_t N, int64_t K, int uc0, int U, int r0,
                                                 int p) {
        static_assert(std::is_same_v<Raw, RawAny>);
        const int lane = tidx() & 63;
        const int slot = lane & (LPR - 1), rip = lane / LPR;
        int64_t row = r0 + p * RPP + rip;
        row = row < N ? row : N - 1;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = slot + LPR * i;
            load_any_kq(raw[p][i], q6, W, N, K, row, uc0 + (u < U ? u : U - 1));
        }
    }

    template <int FMT>
    __device__ __forceinline__ float dot_pass(const XRegs<FMT, LPR, UPL>& xr, int U, int p, int slot) const {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = slot + LPR * i;
            const int uc = u < U ? u : U - 1;
            float c;
            if constexpr (std::is_same_v<Raw, RawAny>) c = dot_any<FMT>(raw[p][i], uc, xr.x[i]);
            else c = dot_reg(raw[p][i], uc, xr.x[i]);
            acc += u < U ? c : 0.f;
        }
        return acc;
    }

    // out[p]: the row sum of pass p, valid in lane sum_lane<LPR>(lane / LPR).
    // side(p) runs after pass p's products (the next stage's loads issued
    // between passes, so the texture unit works while the SIMD computes).
    template <int FMT, class Side>
    __device__ __forceinline__ void dot(const XRegs<FMT, LPR, UPL>& xr, int U, float (&out)[NP], Side side) const {
        // one lane slot for every pass, so the unit-dependent values (scale
        // positions, activation offsets) are formed once, not per pass
        const int slot = (tidx() & 63) & (LPR - 1);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            out[p] = dot_pass<FMT>(xr, U, p, slot);
            side(p);
            pin();
        }
        group_sum<LPR, NP>(out);
    }
    template <int FMT>
    __device__ __forceinline__ void dot(const XRegs<FMT, LPR, UPL>& xr, int U, float (&out)[NP]) const {
        const int slot = (tidx() & 63) & (LPR - 1);
#pragma unroll
        for (int p = 0; p < NP; ++p) out[p] = dot_pass<FMT>(xr, U, p, slot);
        group_sum<LPR, NP>(out);
    }
    // The first np passes only (np wave-uniform): a wave with fewer rows than
    // the task holds skips the products of the passes past its rows.
    template <int FMT>
    __device__ __forceinline__ void dot_n(const XRegs<FMT, LPR, UPL>& xr, int U, int np, float (&out)[NP]) const {
        const int slot = (tidx() & 63) & (LPR - 1);
        np = __builtin_amdgcn_readfirstlane(np);
#pragma unroll
        for (int p = 0; p < NP; ++p) out[p] = p < np ? dot_pass<FMT>(xr, U, p, slot) : 0.f;
        group_sum<LPR, NP>(out);
    }
};

// Two tasks of one format and shape (gate / up) pass by pass, side(p) after each.
template <int FMT, class Raw, int LPR, int UPL, int NP, class Side>
__device__ __forceinline__ void dot_pair(const Task<Raw, LPR, UPL, NP>& ta, const Task<Raw, LPR, UPL, NP>& tb,
                                         const XRegs<FMT, LPR, UPL>& xr, int U, float (&oa)[NP], float (&ob)[NP],
                                         Side side) {
    const int slot = (tidx() & 63) & (LPR - 1);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        oa[p] = ta.template dot_pass<FMT>(xr, U, p, slot);
        ob[p] = tb.template dot_pass<FMT>(xr, U, p, slot);
        side(p);
        pin();
    }
    group_sum<LPR, NP>(oa);
    group_sum<LPR, NP>(ob);
}

// Calls emit(row, value) from the lane holding each row's sum, for rows below
// r_end.
template <int LPR, int NP, class Emit>
__device__ __forceinline__ void emit_rows(int r0, int r_end, const float (&out)[NP], Emit emit) {
    const int lane = tidx() & 63;
    const int g = lane / LPR;
    if (lane != sum_lane<LPR>(g)) return;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int r = r0 + p * (64 / LPR) + g;
        if (r < r_end) emit(r, out[p]);
    }
}

__device__ __forceinline__ void range_of(int n, int parts, int i, int& b, int& e) {
    b = (int)((int64_t)n * i / parts);
    e = (int)((int64_t)n * (i + 1) / parts);
}

// ---- LDS ------------------------------------------------------------------------

// Dynamic LDS after the layer table.  The attention tile is a separate static
// array (see the kernel), so the compiler can tell the tile's LDS-DMA writes
// from the reads of everything here and does not wait for them.
struct Arena {
    float* hv;        // H: the residual (FP32), identical in every workgroup
    uint32_t* xs;     // kmax / 2: swizzled FP16 pairs of the current activation
    float* xsum;      // kmax / 8: sums of 8 consecutive elements
    float* red;       // 64: reduction scratch
    float* rows;      // 256: this workgroup's stage outputs before they are packed into words
    float* att;       // attention scratch (q / k / v of the unit, per-wave areas, part records)
};

__host__ __device__ inline int kmax_of(int H, int fx_max, int slice_o) {
    return std::max(H, std::max(fx_max, slice_o));
}
__host__ __device__ inline size_t att_wave_floats(int hd) { return (size_t)2 * hd + hd + 2 * kTile; }
__host__ __device__ inline size_t att_floats(int hd, int gpu, int Gq) {
    return (size_t)gpu * (Gq + 2) * hd + (size_t)kW * att_wave_floats(hd) + (size_t)kW * (hd + 2) + 2 * kG;
}
__host__ __device__ inline size_t table_bytes(int L) { return ((size_t)L * sizeof(bx_decode_layer) + 15) / 16 * 16; }
__host__ __device__ inline size_t arena_bytes(int H, int kmax, int hd, int gpu, int Gq) {
    return (size_t)H * 4 + (size_t)kmax * 2 + (size_t)(kmax / 8) * 4 + 64 * 4 + 256 * 4 + att_floats(hd, gpu, Gq) * 4;
}
__device__ __forceinline__ Arena make_arena(unsigned char* base, int H, int kmax) {
    Arena r;
    size_t o = 0;
    r.hv = reinterpret_cast<float*>(base + o); o += (size_t)H * 4;
    r.xs = reinterpret_cast<uint32_t*>(base + o); o += (size_t)kmax * 2;
    r.xsum = reinterpret_cast<float*>(base + o); o += (size_t)(kmax / 8) * 4;
    r.red = reinterpret_cast<float*>(base + o); o += 64 * 4;
    r.rows = reinterpret_cast<float*>(base + o); o += 256 * 4;
    r.att = reinterpret_cast<float*>(base + o);
    return r;
}

// One FP16 value (bits v) of element e into the swizzled pairs: group g =
// e / 4 holds dwords 2g = (x0, x2) and 2g + 1 = (x1, x3).
__device__ __forceinline__ void put_swz(uint32_t* xs, int e, uint32_t v) {
    reinterpret_cast<uint16_t*>(xs)[4 * (e >> 2) + 2 * (e & 1) + ((e >> 1) & 1)] = (uint16_t)v;
}

// A thread's norm gammas (8 FP16 values per 256-thread round, H <= 4096),
// requested before the stage's input polls so that their latency hides under
// the hand-off.  Loads past H repeat the first 8 values (issued
// unconditionally, so the compiler counts them exactly).
constexpr int kGammaRounds = 2;
struct GammaRegs {
    u4v g[kGammaRounds];
    __device__ __forceinline__ void load(const void* gamma, int H) {
#pragma unroll
        for (int i = 0; i < kGammaRounds; ++i) {
            const int c = tidx() + i * kT;
            g[i] = gptr<u4v>(gamma)[8 * c < H ? c : 0];
        }
    }
};

// RMSNorm of the residual into the swizzled FP16 activation and its 8-sums:
// x = f16(h * inv * gamma), inv = (mean(h^2) + eps)^-1/2; `ss` is this
// thread's share of sum(h^2) (every element counted by exactly one thread).
__device__ __forceinline__ void norm_to_xs(const Arena& ar, int H, float ss, const GammaRegs& gr, float eps) {
    ss = wave_sum(ss);
    if ((tidx() & 63) == 0) ar.red[tidx() >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kW; ++i) tot += ar.red[i];
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
    for (int i = 0; i < kGammaRounds; ++i) {
        const int c = tidx() + i * kT;
        if (8 * c >= H) break;
        const u4v gm = gr.g[i];
        const float4 v0 = *reinterpret_cast<const float4*>(ar.hv + 8 * c);
        const float4 v1 = *reinterpret_cast<const float4*>(ar.hv + 8 * c + 4);
        const uint32_t h0 = norm_f16(v0.x, inv, h2f(gm.x & 0xffff)), h1 = norm_f16(v0.y, inv, h2f(gm.x >> 16));
        const uint32_t h2 = norm_f16(v0.z, inv, h2f(gm.y & 0xffff)), h3 = norm_f16(v0.w, inv, h2f(gm.y >> 16));
        const uint32_t h4 = norm_f16(v1.x, inv, h2f(gm.z & 0xffff)), h5 = norm_f16(v1.y, inv, h2f(gm.z >> 16));
        const uint32_t h6 = norm_f16(v1.z, inv, h2f(gm.w & 0xffff)), h7 = norm_f16(v1.w, inv, h2f(gm.w >> 16));
        u4v d;
        d.x = h0 | (h2 << 16);
        d.y = h1 | (h3 << 16);
        d.z = h4 | (h6 << 16);
        d.w = h5 | (h7 << 16);
        *reinterpret_cast<u4v*>(ar.xs + 4 * c) = d;
        ar.xsum[c] = ((h2f(h0) + h2f(h2)) + (h2f(h1) + h2f(h3))) + ((h2f(h4) + h2f(h6)) + (h2f(h5) + h2f(h7)));
    }
    __syncthreads();
}

// The residual update of a layer half is the sum of the XCDs' partials (Wo
// over each attention unit's heads, Wd over each FFN slice).  It reaches every
// workgroup in two hops: workgroup (x, r) sums the partials of its own rows
// [r Hr, r Hr + Hr) over the XCDs in xmask, in XCD order, and publishes the
// sum rounded to FP16 (the op path's projection output) through its XCD's L2;
// then every workgroup of XCD x adds the 32 blocks to its copy of h.  The
// first hop crosses XCDs with Hr words per XCD, the second stays in the L2.
__device__ __forceinline__ bool reduce_block(const Args& a, const Arena& ar, const uint64_t* part, uint32_t xmask,
                                             int x, int r, uint32_t tin, uint32_t site, uint64_t* hup,
                                             uint32_t tout) {
    const int Hr = a.H / kR;
    const __amdgpu_buffer_rsrc_t rs = rsrc(part);
    bool ok = true;
    __syncthreads();   // ar.rows may still be read by the previous stage's emit
    const int q0 = __builtin_ctz(xmask);   // XCDs outside xmask poll a copy of the first one's words
    for (int p = tidx(); p < Hr / 2; p += kT) {
        int off[kX];
#pragma unroll
        for (int q = 0; q < kX; ++q) off[q] = (((xmask >> q) & 1u ? q : q0) * a.part_stride + r * Hr + 2 * p) * 8;
        u4v v[kX];
        ok = ok && poll_slots<kX, kCross>(a, rs, off, kX, tin, site, v);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int q = 0; q < kX; ++q) {
            if (!((xmask >> q) & 1u)) continue;
            s0 += __uint_as_float(v[q][0]);
            s1 += __uint_as_float(v[q][2]);
        }
        ar.rows[2 * p] = s0;
        ar.rows[2 * p + 1] = s1;
    }
    if (!__syncthreads_and(ok)) return false;
    uint64_t* out = hup + (int64_t)x * a.hup_stride + r * a.wpart;
    for (int k = tidx(); k < a.wpart; k += kT) {
        uint32_t v[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) v[j] = 3 * k + j < Hr ? f2h(ar.rows[3 * k + j]) : 0u;
        st_local(out + k, word3(tout, v[0], v[1], v[2]));
    }
    return true;
}

// h += the 32 FP16 update blocks of XCD x; ss = this thread's share of sum(h^2).
__device__ __forceinline__ bool apply_update(const Args& a, const Arena& ar, const uint64_t* hup, int x, uint32_t tag,
                                             uint32_t site, float& ss) {
    const int Hr = a.H / kR;
    const FastDivP dw(a.wpart);
    ss = 0.f;
    return poll_vec<2, kLocal>(a, hup + (int64_t)x * a.hup_stride, kR * a.wpart, tag, site,
                               [&](int W, uint32_t lo, uint32_t hi) {
                                   const int rr = dw.div(W), k = W - rr * a.wpart;
#pragma unroll
                                   for (int j = 0; j < 3; ++j) {
                                       if (3 * k + j >= Hr) continue;
                                       const int row = rr * Hr + 3 * k + j;
                                       const float hvv = ar.hv[row] + h2f((uint16_t)fld(lo, hi, j));
                                       ar.hv[row] = hvv;
                                       ss += hvv * hvv;
                                   }
                               });
}

// This workgroup's partial rows [hb, hb + Hr) (ar.rows) as FP32 words.
__device__ __forceinline__ void emit_partial(const Args& a, const Arena& ar, uint64_t* part, int x, int r,
                                             uint32_t tag) {
    const int Hr = a.H / kR;
    uint64_t* out = part + (int64_t)x * a.part_stride + r * Hr;
    for (int i = tidx(); i < Hr; i += kT) st_cross(out + i, word1(tag, __float_as_uint(ar.rows[i])));
}

// ---- attention --------------------------------------------------------------------

// Key splits of a group for context n: at least kMinKeys keys per split until
// smax splits are open, every split non-empty.
__host__ __device__ inline void split_plan(int n, int smax, int& kps, int& S) {
    S = (n + kMinKeys - 1) / kMinKeys;
    if (S > smax) S = smax;
    if (S < 1) S = 1;
    kps = (n + S - 1) / S;
    S = (n + kps - 1) / kps;
}

// Per-lane constants of one head row (pairs p = lane + 64 i): QK-norm gamma
// pairs and RoPE cos / sin of row pos, loaded before q arrives.
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
            c[i] = s[i] = 0.f;
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

// One FP32 head (one wave): per-head RMSNorm with gamma pairs gm (when
// qk_norm), rounded to FP16 as the op path stores it, then RoPE on the FP16
// pairs (rows permuted at load so pair p rotates elements 2p, 2p + 1) ->
// FP16 pairs at dst.
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
    if (qk_norm) inv = 1.0f / sqrtf(wave_sum(ss) / (float)HD + eps);
#pragma unroll
    for (int i = 0; i < kP; ++i) {
        const int p = lane + 64 * i;
        if (p < HD / 2) {
            const float a0 = qk_norm ? h2f(norm_f16(x0[i], inv, h2f(gm[i] & 0xffff))) : r16(x0[i]);
            const float a1 = qk_norm ? h2f(norm_f16(x1[i], inv, h2f(gm[i] >> 16))) : r16(x1[i]);
            const float y0 = f32_fence(__builtin_fmaf(a0, rr.c[i], -f32_fence(a1 * rr.s[i])));
            const float y1 = f32_fence(__builtin_fmaf(a0, rr.s[i], f32_fence(a1 * rr.c[i])));
            dst[p] = pack16(y0, y1);
        }
    }
}

// One 16-byte LDS-DMA copy per lane: lane i's 16 bytes land at lds + 16 i
// (lds is wave-uniform).  ASM issues it from inline assembly (M0 = LDS base);
// no other code in these kernels uses M0, so clobbering it is safe here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool ASM>
__device__ __forceinline__ void dma16(const void* src, void* lds) {
    if constexpr (ASM) {
        const uint32_t base = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base)
                     : "memory", "m0");
    } else {
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
    }
}
#pragma clang diagnostic pop

// Keys [c0, c0 + nk) of one KV head into the LDS tile: K with its 16-byte
// chunks XOR-swizzled by the key (chunk d8 of key j at d8 ^ (j mod HD/8), so
// lanes reading consecutive keys hit distinct banks), V in natural order.
// Slots past nk in the last copy instruction repeat key nk - 1.
template <int HD, bool ASM>
__device__ __forceinline__ void dma_tile(const uint16_t* Kc, const uint16_t* Vc, int64_t kvd, int64_t col0, int c0,
                                         int nk, uint16_t* kt, uint16_t* vt) {
    constexpr int CPK = HD / 8;
    const int ninst = (nk * CPK + 63) / 64;
    const int wave = tidx() >> 6, lane = tidx() & 63;
    for (int i = wave; i < ninst; i += kW) {
        const int slot = 64 * i + lane;
        int j = slot / CPK;
        const int pc = slot % CPK;
        if (j >= nk) j = nk - 1;
        const int64_t row = (int64_t)(c0 + j) * kvd + col0;
        dma16<ASM>(Kc + row + 8 * (pc ^ (j & (CPK - 1))), kt + 512 * i);
        dma16<ASM>(Vc + row + 8 * pc, vt + 512 * i);
    }
}

// This workgroup's attention role for position pos: false when it has none.
struct Split {
    int x, gl, g, s, S, kps, kb, ke;
};
__device__ __forceinline__ bool split_of(const Args& a, int w, int pos, Split& sp) {
    sp.x = w & (kX - 1);
    if (sp.x >= a.nu) return false;
    const int r = w / kX;
    sp.gl = r % a.gpu;
    sp.s = r / a.gpu;
    if (sp.s >= a.smax) return false;
    split_plan(pos + 1, a.smax, sp.kps, sp.S);
    if (sp.s >= sp.S) return false;
    sp.g = sp.x * a.gpu + sp.gl;
    sp.kb = sp.s * sp.kps;
    sp.ke = min(pos + 1, sp.kb + sp.kps);
    return true;
}

template <int HD, bool ASM>
__device__ __forceinline__ void tile_prefetch(const Args& a, int w, const bx_decode_layer& Ly, int pos,
                                              uint16_t* tile) {
    Split sp;
    if (!split_of(a, w, pos, sp)) return;
    dma_tile<HD, ASM>(static_cast<const uint16_t*>(Ly.Kc), static_cast<const uint16_t*>(Ly.Vc), (int64_t)a.nkv * HD,
                      (int64_t)sp.g * HD, sp.kb, min(sp.ke - sp.kb, kTile), tile, tile + kTile * HD);
}

// Row of word W of a unit's q / k / v vector: segment seg, segment row (or -1
// for a padding slot).
__device__ __forceinline__ void qkv_row(const Args& a, int HD, int W, int j, int& seg, int& row) {
    const int Gq = a.nq / a.nkv;
    const int oq = 0, ok = a.aq * a.wq, ov = ok + a.ak * a.wk;
    int base, n, wseg, R;
    if (W < ok) { seg = 0; base = oq; n = a.aq; wseg = a.wq; R = a.gpu * Gq * HD; }
    else if (W < ov) { seg = 1; base = ok; n = a.ak; wseg = a.wk; R = a.gpu * HD; }
    else { seg = 2; base = ov; n = 32 - a.aq - a.ak; wseg = a.wv; R = a.gpu * HD; }
    const int i = (W - base) / wseg, k = (W - base) - i * wseg;
    int rb, re;
    range_of(R, n, i, rb, re);
    row = rb + 3 * k + j;
    if (row >= re) row = -1;
}

// Attention scratch of a split workgroup inside ar.att: the unit's q / k / v
// (FP32), per wave its roped q head, the current key / value rows, scores and
// probabilities, and per wave a partial record (o over HD dims, m, l).
template <int HD>
struct AttScratch {
    float* qraw;   // gpu Gq HD
    float* kraw;   // gpu HD
    float* vraw;   // gpu HD
    float* wv;     // this wave's area
    float* parts;  // kW x (HD + 2)
    __device__ __forceinline__ AttScratch(const Args& a, const Arena& ar) {
        const int Gq = a.nq / a.nkv;
        qraw = ar.att;
        kraw = qraw + a.gpu * Gq * HD;
        vraw = kraw + a.gpu * HD;
        wv = vraw + a.gpu * HD + (tidx() >> 6) * att_wave_floats(HD);
        parts = vraw + a.gpu * HD + kW * att_wave_floats(HD);
    }
    __device__ __forceinline__ uint32_t* q16() const { return reinterpret_cast<uint32_t*>(wv); }
    __device__ __forceinline__ uint32_t* kcur() const { return reinterpret_cast<uint32_t*>(wv) + HD; }
    __device__ __forceinline__ uint32_t* vcur() const { return kcur() + HD / 2; }
    // the wave's key probabilities for P.V (2 kTile floats after q / k / v)
    __device__ __forceinline__ float* pbuf() const { return wv + 2 * HD; }
};

// Stage B of one (group, split): a normalized partial per query head of the
// group over the split's keys -> record words [o (FP16 triples) | m | l].
// Waves work alone: wave w takes part w mod P of the keys for head w / P
// (P = 4 / Gq parts per head), one lane per key for the scores, P.V with two
// head dims per lane; the parts of a head merge in LDS into its record.
template <int HD, bool ASM>
__device__ __forceinline__ bool attention_split(const Args& a, int w, const Arena& ar, uint16_t* tile,
                                                const bx_decode_layer& Ly, int layer, int pos) {
    constexpr int CPK = HD / 8;
    constexpr int W3 = words3(HD);
    Split sp;
    if (!split_of(a, w, pos, sp)) return true;
    const int Gq = a.nq / a.nkv;
    const int wave = tidx() >> 6, lane = tidx() & 63;
    const int P = kW / Gq;                       // key parts per head (Gq <= kW)
    const int part = wave % P, hh = wave / P;    // head of the group this wave serves
    // the split's keys in chunks of one tile (chunk 0 was copied a stage
    // ahead); the current key, when the split holds it, is the last chunk's last
    const int nk = sp.ke - sp.kb, nch = (nk + kTile - 1) / kTile, nlast = nk - (nch - 1) * kTile;
    auto part_of = [&](int cn, int& jb, int& je) {
        const int kpp = (cn + P - 1) / P;
        jb = min(cn, part * kpp);
        je = min(cn, jb + kpp);
    };
    const bool has_cur = sp.ke == pos + 1;
    const int jcur = nlast - 1;
    int jbl, jel;
    part_of(nlast, jbl, jel);
    const bool mine_cur = has_cur && jcur >= jbl && jcur < jel;
    const AttScratch<HD> sc(a, ar);
    uint16_t* kt = tile;
    uint16_t* vt = tile + kTile * HD;
    RopeRegs<HD> rr;
    rr.load(Ly, a.cos_t + (int64_t)pos * (HD / 2), a.sin_t + (int64_t)pos * (HD / 2), a.qk_norm != 0);

    bool ok = poll_vec<2, kLocal>(a, a.qkv + (int64_t)sp.x * a.qkv_stride, a.wqkv, tag_of(a, layer, 0), 10,
                                  [&](int W, uint32_t lo, uint32_t hi) {
#pragma unroll
                                      for (int j = 0; j < 3; ++j) {
                                          int seg, row;
                                          qkv_row(a, HD, W, j, seg, row);
                                          if (row < 0) continue;
                                          float* dst = seg == 0 ? sc.qraw : (seg == 1 ? sc.kraw : sc.vraw);
                                          dst[row] = h2f((uint16_t)fld(lo, hi, j));
                                      }
                                  });
    sub(a, layer, 1);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's tile copies have landed
    if (!__syncthreads_and(ok)) return false;
    sub(a, layer, 2);

    // q head of this wave, and the current key / value for the part holding pos
    const int h = sp.gl * Gq + hh;   // head within the unit
    norm_rope_head<HD>(sc.qraw + h * HD, rr.qg, rr, a.eps, a.qk_norm != 0, sc.q16());
    if (mine_cur) {
        uint32_t* kc = sc.kcur();
        uint32_t* vc = sc.vcur();
        norm_rope_head<HD>(sc.kraw + sp.gl * HD, rr.kg, rr, a.eps, a.qk_norm != 0, kc);
        for (int p = lane; p < HD / 2; p += 64)
            vc[p] = pack16(sc.vraw[sp.gl * HD + 2 * p], sc.vraw[sp.gl * HD + 2 * p + 1]);
        if (hh == 0) {   // the KV-cache row, once per group
            const int64_t kvd = (int64_t)a.nkv * HD;
            uint16_t* Kw = static_cast<uint16_t*>(Ly.Kc) + (int64_t)pos * kvd + (int64_t)sp.g * HD;
            uint16_t* Vw = static_cast<uint16_t*>(Ly.Vc) + (int64_t)pos * kvd + (int64_t)sp.g * HD;
            for (int p = lane; p < HD / 2; p += 64) {
                gptr_w<uint32_t>(Kw)[p] = kc[p];
                gptr_w<uint32_t>(Vw)[p] = vc[p];
            }
        }
    }

    sub(a, layer, 3);
    const float scale = 1.0f / sqrtf((float)HD);
    const uint32_t* q = sc.q16();
    float* pb = sc.pbuf();
    // this wave's running maximum and sum, and its unnormalized P.V with dims
    // 2 lane, 2 lane + 1; a chunk's probabilities are taken against the
    // running maximum and what came before is rescaled when it grows (one
    // chunk: the single-pass softmax of the wave's keys)
    float Mw = -INFINITY, Lw = 0.f, o0 = 0.f, o1 = 0.f;
    // one chunk of cn keys in the tile; last: it holds the current key
    auto chunk = [&](int cn, bool last) __attribute__((always_inline)) {
        int jb, je;
        part_of(cn, jb, je);
        if (mine_cur && last) {
            // the current key / value replace the (stale) cache row in the tile
            const uint32_t* kc = sc.kcur();
            const uint32_t* vc = sc.vcur();
            for (int d8 = lane; d8 < CPK; d8 += 64) {
                *reinterpret_cast<u4v*>(kt + jcur * HD + 8 * (d8 ^ (jcur & (CPK - 1)))) =
                    *reinterpret_cast<const u4v*>(kc + 4 * d8);
                *reinterpret_cast<u4v*>(vt + jcur * HD + 8 * d8) = *reinterpret_cast<const u4v*>(vc + 4 * d8);
            }
        }
        // scores of this wave's keys (lane t: keys jb + t, jb + 64 + t)
        const int nkw = je - jb;
        float sv[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int t = lane + 64 * hb;
            sv[hb] = -INFINITY;
            if (64 * hb < nkw) {
                const int jr = jb + (t < nkw ? t : nkw - 1);
                const uint16_t* kr = kt + jr * HD;
                float acc = 0.f, acc2 = 0.f;
#pragma unroll
                for (int d0 = 0; d0 < CPK; d0 += 8) {
                    u4v kk[8], qv[8];
#pragma unroll
                    for (int c8 = 0; c8 < 8; ++c8) {
                        kk[c8] = *reinterpret_cast<const u4v*>(kr + 8 * ((d0 + c8) ^ (jr & (CPK - 1))));
                        qv[c8] = *reinterpret_cast<const u4v*>(q + 4 * (d0 + c8));
                    }
                    pin();
#pragma unroll
                    for (int c8 = 0; c8 < 8; ++c8) {
                        acc = dot2(qv[c8].x, kk[c8].x, acc);
                        acc2 = dot2(qv[c8].y, kk[c8].y, acc2);
                        acc = dot2(qv[c8].z, kk[c8].z, acc);
                        acc2 = dot2(qv[c8].w, kk[c8].w, acc2);
                    }
                }
                if (t < nkw) sv[hb] = (acc + acc2) * scale;
            }
        }
        const float M = fmaxf(Mw, wave_max(fmaxf(sv[0], sv[1])));
        const float al = Mw == -INFINITY ? 0.f : __expf(Mw - M);
        float pv[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) pv[hb] = lane + 64 * hb < nkw ? r16(__expf(sv[hb] - M)) : 0.f;
        Lw = Lw * al + wave_sum(pv[0] + pv[1]);
        Mw = M;
        // the probabilities go through LDS: the P.V loop then reads four keys'
        // worth per broadcast load, where a readlane per key costs the wait
        // states before its scalar result can feed the multiply (the wave's own
        // LDS writes complete before its later reads)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
            if (lane + 64 * hb < nkw) pb[lane + 64 * hb] = pv[hb];
        o0 *= al;
        o1 *= al;
        const uint16_t* vcol = vt + jb * HD + 2 * (2 * lane < HD ? lane : 0);
        for (int t0 = 0; t0 < nkw; t0 += 8) {
            uint32_t vv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) vv[u] = *reinterpret_cast<const uint32_t*>(vcol + min(t0 + u, nkw - 1) * HD);
            const u4v pa = *reinterpret_cast<const u4v*>(pb + t0), pc = *reinterpret_cast<const u4v*>(pb + t0 + 4);
            pin();
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float p = t0 + u < nkw ? __uint_as_float(u < 4 ? pa[u] : pc[u - 4]) : 0.f;
                o0 += p * h2f(vv[u] & 0xffff);
                o1 += p * h2f(vv[u] >> 16);
            }
        }
    };
    // chunk 0 was copied a stage ahead (straight-line: the running state
    // starts empty); further chunks replace it in the tile
    chunk(nch == 1 ? nlast : kTile, nch == 1);
    for (int c = 1; c < nch; ++c) {
        const int cn = c == nch - 1 ? nlast : kTile;
        __syncthreads();   // every wave is done with the previous chunk
        dma_tile<HD, ASM>(static_cast<const uint16_t*>(Ly.Kc), static_cast<const uint16_t*>(Ly.Vc),
                          (int64_t)a.nkv * HD, (int64_t)sp.g * HD, sp.kb + c * kTile, cn, kt, vt);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        chunk(cn, c == nch - 1);
    }
    sub(a, layer, 4);
    // this wave's part: o (unnormalized), m, l (a part without keys has m =
    // -inf, l = 0)
    float* pr = sc.parts + wave * (HD + 2);
    if (2 * lane < HD) {
        pr[2 * lane] = o0;
        pr[2 * lane + 1] = o1;
    }
    if (lane == 0) {
        pr[HD] = Mw;
        pr[HD + 1] = Lw;
    }
    __syncthreads();
    sub(a, layer, 5);
    // records of the group's heads: o / l over the merged parts (FP16), m, l
    const uint32_t tout = tag_of(a, layer, 1);
    uint64_t* rbase = a.recw + (int64_t)sp.x * a.rec_stride + (int64_t)((sp.gl * a.smax + sp.s) * Gq) * a.rec;
    for (int t = tidx(); t < Gq * a.rec; t += kT) {
        const int hd_ = t / a.rec, k = t - hd_ * a.rec;
        float mm = -INFINITY;
        for (int p = 0; p < P; ++p) mm = fmaxf(mm, sc.parts[(hd_ * P + p) * (HD + 2) + HD]);
        float wsum = 0.f, wp[kW];
#pragma unroll
        for (int p = 0; p < kW; ++p) {
            wp[p] = 0.f;
            if (p < P) {
                const float* q2 = sc.parts + (hd_ * P + p) * (HD + 2);
                wp[p] = q2[HD + 1] > 0.f ? __expf(q2[HD] - mm) : 0.f;
                wsum += wp[p] * q2[HD + 1];
            }
        }
        uint64_t wd;
        if (k < W3) {
            uint32_t v3[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int d = 3 * k + j;
                float o = 0.f;
                if (d < HD)
#pragma unroll
                    for (int p = 0; p < kW; ++p)
                        if (p < P) o += wp[p] * sc.parts[(hd_ * P + p) * (HD + 2) + d];
                v3[j] = d < HD ? f2h(o / wsum) : 0u;
            }
            wd = word3(tout, v3[0], v3[1], v3[2]);
        } else if (k == W3) {
            wd = word1(tout, __float_as_uint(mm));
        } else if (k == W3 + 1) {
            wd = word1(tout, __float_as_uint(wsum));
        } else {
            wd = word1(tout, 0u);
        }
        st_local(rbase + t, wd);
    }
    sub(a, layer, 6);
    return true;
}

// Stage C input: every record of the unit -> the attention output of its
// gpu Gq heads, FP16 (the op path's attention output), into the swizzled
// activation of the Wo slice, and its 8-sums.  Records go to LDS over the
// idle attention tile (recs[(head S + s)(HD + 2) + d]).
template <int HD>
__device__ __forceinline__ bool combine(const Args& a, int x, const Arena& ar, float* recs, int layer, int pos) {
    constexpr int W3 = words3(HD);
    const int Gq = a.nq / a.nkv, heads = a.gpu * Gq;
    int kps, S;
    split_plan(pos + 1, a.smax, kps, S);
    const uint32_t tag = tag_of(a, layer, 1);
    const FastDivP drec(a.rec);
    for (int gl = 0; gl < a.gpu; ++gl) {
        const uint64_t* src = a.recw + (int64_t)x * a.rec_stride + (int64_t)(gl * a.smax * Gq) * a.rec;
        const bool ok = poll_vec<4, kLocal>(a, src, S * Gq * a.rec, tag, 13, [&](int W, uint32_t lo, uint32_t hi) {
            const int q = drec.div(W), k = W - q * a.rec;
            const int s = q / Gq, h = gl * Gq + (q - s * Gq);
            float* r = recs + (h * S + s) * (HD + 2);
            if (k < W3) {
#pragma unroll
                for (int j = 0; j < 3; ++j)
                    if (3 * k + j < HD) r[3 * k + j] = h2f((uint16_t)fld(lo, hi, j));
            } else if (k == W3) {
                r[HD] = __uint_as_float(lo);
            } else if (k == W3 + 1) {
                r[HD + 1] = __uint_as_float(lo);
            }
        });
        if (!__syncthreads_and(ok)) return false;
    }
    sub(a, layer, 15);
    // weights per (head, split), exp(m_s - M) l_s / sum: one wave per head, one lane per split
    float* wts = ar.att;   // heads x S
    {
        const int lane = tidx() & 63;
        for (int h = tidx() >> 6; h < heads; h += kW) {
            float m = -INFINITY, l = 0.f;
            if (lane < S) {
                m = recs[(h * S + lane) * (HD + 2) + HD];
                l = recs[(h * S + lane) * (HD + 2) + HD + 1];
            }
            const float M = wave_max(m);
            const float wgt = lane < S && l > 0.f ? __expf(m - M) * l : 0.f;
            const float tot = wave_sum(wgt);
            if (lane < S) wts[h * S + lane] = wgt / tot;
        }
    }
    __syncthreads();
    sub(a, layer, 16);
    // output element (head h, dim d) -> FP16 -> swizzled activation
    for (int t = tidx(); t < heads * HD; t += kT) {
        const int h = t / HD, d = t - h * HD;
        const float* r0 = recs + h * S * (HD + 2) + d;
        const float* w0 = wts + h * S;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        int s = 0;
        for (; s + 4 <= S; s += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) o[u] += w0[s + u] * r0[(s + u) * (HD + 2)];
        }
        for (; s < S; ++s) o[0] += w0[s] * r0[s * (HD + 2)];
        put_swz(ar.xs, h * HD + d, f2h((o[0] + o[1]) + (o[2] + o[3])));
    }
    __syncthreads();
    sums8_from_lds(ar.xs, heads * HD, ar.xsum);
    __syncthreads();
    return true;
}

// ---- the kernel ------------------------------------------------------------------------

// Rows of a wave's share of [b, e) (contiguous, in wave order).
__device__ __forceinline__ void wave_share(int b, int e, int& wb, int& we) {
    const int wave = tidx() >> 6;
    wb = b + (int)((int64_t)(e - b) * wave / kW);
    we = b + (int)((int64_t)(e - b) * (wave + 1) / kW);
}

// Pack rows [rb, re) of this workgroup's stage outputs (vals[row - rb], in
// LDS) into nw words (three rows each, padding slots 0) at out.
template <bool CROSS>
__device__ __forceinline__ void emit_words(const float* vals, int rb, int re, int nw, uint64_t* out, uint32_t tag) {
    for (int k = tidx(); k < nw; k += kT) {
        uint32_t v[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int r = rb + 3 * k + j;
            v[j] = r < re ? f2h(vals[r - rb]) : 0u;
        }
        const uint64_t wd = word3(tag, v[0], v[1], v[2]);
        if (CROSS) st_cross(out + k, wd);
        else st_local(out + k, wd);
    }
}

// FFN slice [fb, fe) of XCD x: F in blocks of fblk, blocks spread evenly.
__device__ __forceinline__ void ffn_slice(const Args& a, int x, int& fb, int& fe) {
    const int nb = a.F / a.fblk;
    fb = (int)((int64_t)nb * x / kX) * a.fblk;
    fe = (int)((int64_t)nb * (x + 1) / kX) * a.fblk;
}
__device__ __forceinline__ uint32_t ffn_mask(const Args& a) {
    uint32_t m = 0;
    for (int x = 0; x < kX; ++x) {
        int fb, fe;
        ffn_slice(a, x, fb, fe);
        if (fe > fb) m |= 1u << x;
    }
    return m;
}

// Template parameters: formats of q / k (FQ), v (FV, or FV2 in some layers;
// -1: none), o, gate / up, down (FD / FD2), lm_head (FH); head_dim; and per
// stage the lanes per row, units per lane and passes of a wave's task: A
// (q / k / v, K = H), C (Wo, K = the unit's columns), D (gate / up, K = H),
// E (Wd, K = the FFN slice), H (lm_head, K = H).
template <int FQ, int FV, int FV2, int FO, int FGU, int FD, int FD2, int FH, int HD, int LA, int UA, int NA, int LC,
          int UC, int NC, int LD, int UD, int ND, int LE, int UE, int NE, int LH, int UH, int NH, int OPT>
__global__ __launch_bounds__(kT, 1) void persist2_kernel(Args a) {
    constexpr bool kLateReq = (OPT & kLate) != 0, kAsm = (OPT & kAsmDma) != 0;
    extern __shared__ __align__(16) unsigned char dyn[];
    // The attention tile (keys then values), filled by LDS-DMA one layer ahead;
    // stage C reuses it for the split records.
    __shared__ __align__(16) uint16_t tile[(2 * kTile * HD * 2 > kMaxGq / 2 * kR * (HD + 2) * 4 + 4096
                                                ? 2 * kTile * HD * 2
                                                : kMaxGq / 2 * kR * (HD + 2) * 4 + 4096) /
                                           2];
    const int H = a.H;
    bx_decode_layer* const lt = reinterpret_cast<bx_decode_layer*>(dyn);
    for (int i = tidx(); i < a.L * (int)(sizeof(bx_decode_layer) / 8); i += kT)
        reinterpret_cast<uint64_t*>(dyn)[i] = gptr<uint64_t>(a.layers)[i];
    const int Gq = a.nq / a.nkv;
    const int slice_o = a.gpu * Gq * HD;
    int fxmax = 0;
    for (int x = 0; x < kX; ++x) {
        int fb, fe;
        ffn_slice(a, x, fb, fe);
        fxmax = max(fxmax, fe - fb);
    }
    const int kmax = max(H, max(fxmax, slice_o));
    const Arena ar = make_arena(dyn + table_bytes(a.L), H, kmax);
    const int lane = tidx() & 63;
    const int tok = a.scal[0], pos = a.scal[1];
    stamp(a, 0);
    // this workgroup's XCD and its rank there (an atomic on the XCD's L2, one
    // counter per epoch, zeroed by bx_persist_ws_init): logical id x + 8 rank
    const int x = (int)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 7u);
    int* rank_lds = reinterpret_cast<int*>(ar.red + 32);
    if (tidx() == 0)
        *rank_lds = (int)__hip_atomic_fetch_add(a.ctrl + kCtrlWords + (a.epoch & 63u) * kX + x, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
    __syncthreads();
    const int r = *rank_lds;
    if (r >= kR) {   // more than 32 workgroups on this XCD: the partition cannot hold
        if (tidx() == 0) raise_abort(a, kSiteXcd);
        return;
    }
    const int w = x + kX * r;
    if (a.trace && tidx() == 0) a.trace[(size_t)blockIdx.x * kTraceSlots + 1000] = (uint64_t)w;   // logical id
    // embedding row -> h
    for (int i = tidx(); i < H; i += kT) ar.hv[i] = h2f(a.embed[(int64_t)tok * H + i]);
    __syncthreads();

    const uint32_t xmask_o = (1u << a.nu) - 1u, xmask_d = ffn_mask(a);
    const bool unit = x < a.nu;
    const int Hr = H / kR;
    const int hb = r * Hr, he = hb + Hr;                       // residual rows of Wo / Wd (partials)
    int fb, fe;
    ffn_slice(a, x, fb, fe);
    const int Fx = fe - fb;
    int gb, ge;                                                 // gate / up rows (absolute)
    range_of(Fx, kR, r, gb, ge);
    gb += fb;
    ge += fb;
    // stage A segment of this workgroup
    int seg, si, sn, sR, srow0;
    if (r < a.aq) { seg = 0; si = r; sn = a.aq; sR = a.gpu * Gq * HD; srow0 = x * sR; }
    else if (r < a.aq + a.ak) { seg = 1; si = r - a.aq; sn = a.ak; sR = a.gpu * HD; srow0 = x * sR; }
    else { seg = 2; si = r - a.aq - a.ak; sn = a.av; sR = a.gpu * HD; srow0 = x * sR; }
    int arb, are;
    range_of(sR, sn, si, arb, are);
    const int woff = seg == 0 ? si * a.wq : (seg == 1 ? a.aq * a.wq + si * a.wk : a.aq * a.wq + a.ak * a.wk + si * a.wv);
    const int wseg = seg == 0 ? a.wq : (seg == 1 ? a.wk : a.wv);
    const int aN = seg == 0 ? a.nq * HD : a.nkv * HD;
    int awb, awe, cwb, cwe, dwb, dwe, ewb, ewe;
    wave_share(arb, are, awb, awe);
    wave_share(hb, he, cwb, cwe);
    wave_share(gb, ge, dwb, dwe);
    wave_share(hb, he, ewb, ewe);
    constexpr int RA = NA * (64 / LA), RC = NC * (64 / LC), RD = ND * (64 / LD), RE = NE * (64 / LE);
    const int UAn = H / 32, UCn = slice_o / 32, UEn = Fx / 32;

    using RawA = std::conditional_t<(FV2 < 0 && FV == FQ), typename RawOf<FQ>::T, RawAny>;
    // run-time formats limited to Q4_K / Q6_K take the branch-free requests
    constexpr auto kq = [](int f) { return f < 0 || f == FMT_Q4_K || f == FMT_Q6_K; };
    constexpr bool kAnyA = std::is_same_v<RawA, RawAny> && kq(FQ) && kq(FV) && kq(FV2);
    constexpr bool kAnyE = std::is_same_v<RawFor<FD, FD2>, RawAny> && kq(FD) && kq(FD2);
    Task<RawA, LA, UA, NA> ta;
    Task<typename RawOf<FO>::T, LC, UC, NC> tc;
    Task<typename RawOf<FGU>::T, LD, UD, ND> tg, tu;
    Task<RawFor<FD, FD2>, LE, UE, NE> te;
    auto a_fmt = [&](const bx_decode_layer& Ly) { return seg == 2 ? Ly.type_v : FQ; };
    const void* const* a_mat = seg == 0 ? &lt[0].Wq : (seg == 1 ? &lt[0].Wk : &lt[0].Wv);
    const size_t a_mat_off = (const char*)a_mat - (const char*)&lt[0];
    auto a_w = [&](const bx_decode_layer& Ly) {
        return *reinterpret_cast<const void* const*>(reinterpret_cast<const char*>(&Ly) + a_mat_off);
    };
    // pass p of the q / k / v block of layer Ly (rows clamped: a workgroup
    // without rows loads harmless copies, so the loads stay unconditional)
    auto load_a_pass = [&](const bx_decode_layer& Ly, int p, int zl) {
        const int f = a_fmt(Ly);
        if constexpr (kAnyA) {
            ta.load_pass_kq(f == FMT_Q6_K, a_w(Ly), aN, H, 0, UAn, srow0 + awb + zl, p);
        } else {
            if (seg != 2 || f == FQ) ta.template load_pass<FQ>(a_w(Ly), aN, H, 0, UAn, srow0 + awb + zl, p);
            else if (f == FV) ta.template load_pass<FV>(a_w(Ly), aN, H, 0, UAn, srow0 + awb + zl, p);
            else if constexpr (FV2 >= 0) ta.template load_pass<FV2>(a_w(Ly), aN, H, 0, UAn, srow0 + awb + zl, p);
        }
    };
    const int uc_o = (min(x, a.nu - 1) * slice_o) / 32;
    auto load_d = [&](const bx_decode_layer& Ly, int zl) {
        tg.template load<FGU>(Ly.Wg, a.F, H, 0, UAn, dwb + zl);
        tu.template load<FGU>(Ly.Wu, a.F, H, 0, UAn, dwb + zl);
    };
    auto load_e_pass = [&](const void* Wd, int type_down, int p, int zl) {
        if constexpr (kAnyE) {
            te.load_pass_kq(type_down == FMT_Q6_K, Wd, H, a.F, fb / 32, UEn, ewb + zl, p);
        } else {
            if (type_down == FD) te.template load_pass<FD>(Wd, H, a.F, fb / 32, UEn, ewb + zl, p);
            else if constexpr (FD2 >= 0) te.template load_pass<FD2>(Wd, H, a.F, fb / 32, UEn, ewb + zl, p);
        }
    };

#pragma unroll
    for (int p = 0; p < NA; ++p) load_a_pass(lt[0], p, opaque_zero());
    tile_prefetch<HD, kAsm>(a, w, lt[0], pos, tile);
    pin();

    for (int l = 0; l < a.L; ++l) {
        const bx_decode_layer& Ly = lt[l];
        const bx_decode_layer& Ln = lt[min(l + 1, a.L - 1)];
        const int zl = opaque_zero();
        const int sl = 1 + 9 * l;
        // ---- A: residual, norm, q / k / v rows; the Wo and gate / up blocks
        // are requested between the passes
        {
            GammaRegs gr;
            gr.load(Ly.in_ln, H);
            float ss = 0.f;
            if (l > 0) {
                if (!reduce_block(a, ar, a.pdn + zl, xmask_d, x, r, tag_of(a, l - 1, 4), 1, a.hupd + zl,
                                  tag_of(a, l - 1, 6)))
                    return;
                sub(a, l, 0);
                if (!apply_update(a, ar, a.hupd + zl, x, tag_of(a, l - 1, 6), 7, ss)) return;
                sub(a, l, 7);
            } else {
                for (int i = tidx(); i < H; i += kT) ss += ar.hv[i] * ar.hv[i];
            }
            __syncthreads();
            norm_to_xs(ar, H, ss, gr, a.eps);
            stamp(a, sl + 0);
            // Wo rows stream while q / k / v are computed and travel (kLate:
            // requested after the q / k / v words are out)
            if (!kLateReq && unit) tc.template load<FO>(Ly.Wo, H, a.nq * HD, uc_o + zl, UCn, cwb);
            pin();
            sub(a, l, 8);
            if (unit && awb < awe) {
                auto run = [&](auto fmt_tag) {
                    constexpr int F = decltype(fmt_tag)::value;
                    XRegs<F, LA, UA> xr;
                    xr.load(ar.xs, ar.xsum, UAn);
                    for (int t0 = awb; t0 < awe; t0 += RA) {
                        float o[NA];
                        if (t0 != awb) ta.template load<F>(a_w(Ly), aN, H, 0, UAn, srow0 + t0 + zl);
                        // a segment's rows spread over its workgroups' waves, so a
                        // wave (v rows: Q6_K, fewer per workgroup) may hold fewer
                        // rows than the task's passes
                        ta.template dot_n<F>(xr, UAn, (awe - t0 + (64 / LA) - 1) / (64 / LA), o);
                        emit_rows<LA, NA>(t0, awe, o, [&](int row, float v) { ar.rows[row - arb] = v; });
                    }
                };
                const int f = a_fmt(Ly);
                if (seg != 2 || f == FQ) run(std::integral_constant<int, FQ>{});
                else if (f == FV) run(std::integral_constant<int, FV>{});
                else if constexpr (FV2 >= 0) run(std::integral_constant<int, FV2>{});
            }
            sub(a, l, 9);
            __syncthreads();
            if (unit)
                emit_words<false>(ar.rows, arb, are, wseg, a.qkv + (int64_t)x * a.qkv_stride + woff + zl,
                                  tag_of(a, l, 0));
            if (kLateReq && unit) tc.template load<FO>(Ly.Wo, H, a.nq * HD, uc_o + zl, UCn, cwb);
            pin();
        }
        stamp(a, sl + 1);
        // ---- B: attention splits
        if (!__syncthreads_and(attention_split<HD, kAsm>(a, w, ar, tile, Ly, l, pos))) return;
        stamp(a, sl + 2);
        // ---- C: combine, Wo partial
        if (unit) {
            if (!combine<HD>(a, x, ar, reinterpret_cast<float*>(tile), l, pos)) return;
            stamp(a, sl + 3);
            // gate / up rows stream while the Wo partials travel (before the
            // Wo dots, or with kLate after the partials are out)
            if (!kLateReq) load_d(Ly, zl);
            pin();
            sub(a, l, 17);
            {
                XRegs<FO, LC, UC> xr;
                xr.load(ar.xs, ar.xsum, UCn);
                for (int t0 = cwb; t0 < cwe; t0 += RC) {
                    if (t0 != cwb) tc.template load<FO>(Ly.Wo, H, a.nq * HD, uc_o, UCn, t0 + zl);
                    float o[NC];
                    tc.template dot<FO>(xr, UCn, o);
                    emit_rows<LC, NC>(t0, cwe, o, [&](int row, float v) { ar.rows[row - hb] = v; });
                }
            }
            sub(a, l, 18);
            __syncthreads();
            emit_partial(a, ar, a.pwo + zl, x, r, tag_of(a, l, 2));
            if (kLateReq) load_d(Ly, zl);
            pin();
        } else {
            load_d(Ly, zl);
            pin();
        }
        stamp(a, sl + 4);
        // ---- D: residual, norm, gate / up rows of the slice; the Wd block is
        // requested between the passes
        {
            GammaRegs gr;
            gr.load(Ly.post_ln, H);
            float ss = 0.f;
            if (!reduce_block(a, ar, a.pwo + zl, xmask_o, x, r, tag_of(a, l, 2), 3, a.hupo + zl, tag_of(a, l, 5)))
                return;
            sub(a, l, 10);
            if (!apply_update(a, ar, a.hupo + zl, x, tag_of(a, l, 5), 8, ss)) return;
            sub(a, l, 11);
            __syncthreads();
            norm_to_xs(ar, H, ss, gr, a.eps);
            stamp(a, sl + 5);
            // E's matrix and format, read from the LDS table here: with global
            // stores and loads both outstanding the compiler waits for all of
            // them before a dependent use, so a table read just before a late
            // request, after the SwiGLU words' stores, would wait for those
            const void* const e_w = Ly.Wd;
            const int e_t = Ly.type_down;
            pin();
            // Wd rows stream while gate / up are computed and travel (kLate:
            // requested after the SwiGLU words are out)
            if (!kLateReq) {
#pragma unroll
                for (int p = 0; p < NE; ++p) load_e_pass(e_w, e_t, p, zl);
            }
            pin();
            sub(a, l, 13);
            if (dwb < dwe) {
                XRegs<FGU, LD, UD> xr;
                xr.load(ar.xs, ar.xsum, UAn);
                for (int t0 = dwb; t0 < dwe; t0 += RD) {
                    float og[ND], ou[ND];
                    if (t0 != dwb) {
                        tg.template load<FGU>(Ly.Wg, a.F, H, 0, UAn, t0 + zl);
                        tu.template load<FGU>(Ly.Wu, a.F, H, 0, UAn, t0 + zl);
                    }
                    tg.template dot<FGU>(xr, UAn, og);
                    tu.template dot<FGU>(xr, UAn, ou);
#pragma unroll
                    for (int p = 0; p < ND; ++p) {
                        // the op path's roundings: f16(f16(silu(f16(g))) * f16(u))
                        const float g16 = r16(og[p]), u16 = r16(ou[p]);
                        og[p] = r16(silu_f32(g16)) * u16;
                    }
                    emit_rows<LD, ND>(t0, dwe, og, [&](int row, float v) { ar.rows[row - gb] = v; });
                }
            }
            sub(a, l, 12);
            __syncthreads();
            emit_words<false>(ar.rows, gb, ge, a.wact, a.act + (int64_t)x * a.act_stride + r * a.wact + zl,
                              tag_of(a, l, 3));
            if (kLateReq) {
#pragma unroll
                for (int p = 0; p < NE; ++p) load_e_pass(e_w, e_t, p, zl);
            }
            pin();
            sub(a, l, 14);
        }
        stamp(a, sl + 6);
        // ---- E: the slice's SwiGLU output, Wd partial; the next layer's q / k /
        // v block is requested between the passes
        {
            const int nw = kR * a.wact;
            const FastDivP dwa(a.wact);
            const bool ok = poll_vec<2, kLocal>(
                a, a.act + (int64_t)x * a.act_stride + zl, nw, tag_of(a, l, 3), 4, [&](int W, uint32_t lo, uint32_t hi) {
                    const int rr = dwa.div(W), k = W - rr * a.wact;
                    int b0, e0;
                    range_of(Fx, kR, rr, b0, e0);
#pragma unroll
                    for (int j = 0; j < 3; ++j) {
                        const int e = b0 + 3 * k + j;
                        if (e < e0) put_swz(ar.xs, e, fld(lo, hi, j));
                    }
                });
            if (!__syncthreads_and(ok)) return;
            sub(a, l, 31);
            sums8_from_lds(ar.xs, Fx, ar.xsum);
            __syncthreads();
            stamp(a, sl + 7);
            auto run = [&](auto fmt_tag) {
                constexpr int F = decltype(fmt_tag)::value;
                XRegs<F, LE, UE> xr;
                xr.load(ar.xs, ar.xsum, UEn);
                for (int t0 = ewb; t0 < ewe; t0 += RE) {
                    float o[NE];
                    if (t0 != ewb) te.template load<F>(Ly.Wd, H, a.F, fb / 32, UEn, t0 + zl);
                    te.template dot<F>(xr, UEn, o);
                    emit_rows<LE, NE>(t0, ewe, o, [&](int row, float v) { ar.rows[row - hb] = v; });
                }
            };
            if (Ly.type_down == FD) run(std::integral_constant<int, FD>{});
            else if constexpr (FD2 >= 0) run(std::integral_constant<int, FD2>{});
            sub(a, l, 30);
            __syncthreads();
            emit_partial(a, ar, a.pdn + zl, x, r, tag_of(a, l, 4));
            sub(a, l, 32);
        }
        // the next layer's q / k / v rows, then its attention tile, stream
        // while the down partials travel (the tile's LDS-DMA goes last: the
        // first LDS access after it waits for every load still outstanding,
        // and the next poll waits for those anyway)
        if (l + 1 < a.L) {
#pragma unroll
            for (int p = 0; p < NA; ++p) load_a_pass(Ln, p, zl);
            tile_prefetch<HD, kAsm>(a, w, Ln, pos, tile);
        }
        pin();
        sub(a, l, 33);
        stamp(a, sl + 8);
    }

    // ---- head: residual, final norm, lm_head rows, per-workgroup argmax
    const int sh = 1 + 9 * a.L;
    int vb, ve;
    range_of(a.V, kG, w, vb, ve);
    int hwb, hwe;
    wave_share(vb, ve, hwb, hwe);
    float best = -INFINITY;
    int besti = -1;
    {
        constexpr int RH = NH * (64 / LH);
        using Raw = typename RawOf<FH>::T;
        Raw b0[NH][UH], b1[NH][UH];
        const int slot = lane & (LH - 1), rip = lane / LH;
        auto load = [&](Raw (&b)[NH][UH], int r0) {
#pragma unroll
            for (int p = 0; p < NH; ++p) {
                int64_t row = r0 + p * (64 / LH) + rip;
                row = row < a.V ? row : a.V - 1;
#pragma unroll
                for (int i = 0; i < UH; ++i) {
                    const int u = slot + LH * i;
                    b[p][i] = load_unit<FH>(a.lm_head, a.V, H, row, u < UAn ? u : UAn - 1);
                }
            }
        };
        if (hwb < hwe) load(b0, hwb);
        pin();
        GammaRegs gr;
        gr.load(a.final_norm, H);
        float ss = 0.f;
        if (!reduce_block(a, ar, a.pdn, xmask_d, x, r, tag_of(a, a.L - 1, 4), 5, a.hupd, tag_of(a, a.L - 1, 6)))
            return;
        if (!apply_update(a, ar, a.hupd, x, tag_of(a, a.L - 1, 6), 9, ss)) return;
        __syncthreads();
        norm_to_xs(ar, H, ss, gr, a.eps);
        stamp(a, sh + 0);
        XU xu[UH];
#pragma unroll
        for (int i = 0; i < UH; ++i) {
            const int u = slot + LH * i;
            xu[i] = load_xu<FH == FMT_F16 ? FMT_Q8_0 : FH>(ar.xs, ar.xsum, u < UAn ? u : UAn - 1);
        }
        pin();
        auto dot = [&](const Raw (&b)[NH][UH], int r0) {
            float o[NH];
#pragma unroll
            for (int p = 0; p < NH; ++p) {
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < UH; ++i) {
                    const int u = slot + LH * i;
                    const float c = dot_reg(b[p][i], u < UAn ? u : UAn - 1, xu[i]);
                    acc += u < UAn ? c : 0.f;
                }
                o[p] = acc;
            }
            group_sum<LH, NH>(o);
            emit_rows<LH, NH>(r0, hwe, o, [&](int row, float v) {
                const uint16_t h16 = f2h(v);
                tile[row - vb] = h16;
                const float q = h2f(h16);
                if (besti < 0 || q > best || (q == best && row < besti)) {
                    best = q;
                    besti = row;
                }
            });
        };
        // Both buffers' requests are unconditional (past the wave's rows they
        // re-read its current block, which the L2 holds): a request on one
        // branch only would make the compiler's wait for the other buffer
        // cover every load in flight.
        for (int t = hwb; t < hwe; t += 2 * RH) {
            const int t1 = t + RH;
            load(b1, t1 < hwe ? t1 : t);
            __builtin_amdgcn_sched_barrier(0);   // the requests go out before the other buffer's math
            dot(b0, t);
            if (t1 >= hwe) break;
            load(b0, t1 + RH < hwe ? t1 + RH : t1);
            __builtin_amdgcn_sched_barrier(0);
            dot(b1, t1);
        }
    }
    // The logits leave through LDS after the loop: a global store inside it
    // would leave stores and loads outstanding together, and the compiler then
    // makes each row block's dot wait for every load in flight, the other
    // buffer's included.
    __syncthreads();
    for (int i = tidx(); i < ve - vb; i += kT) a.logits[vb + i] = tile[i];
    stamp(a, sh + 1);
    // workgroup argmax: every lane holds its best (lowest index among equals)
    {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(besti, off, 64);
            if (oi >= 0 && (besti < 0 || ov > best || (ov == best && oi < besti))) {
                best = ov;
                besti = oi;
            }
        }
    }
    float* rv = ar.red;
    int* ri = reinterpret_cast<int*>(ar.red + 8);
    __syncthreads();
    if (lane == 0) {
        rv[tidx() >> 6] = best;
        ri[tidx() >> 6] = besti;
    }
    __syncthreads();
    const uint32_t tc_ = tag_of(a, a.L, 0);
    if (tidx() == 0) {
        float bv = -INFINITY;
        int bi = -1;
        for (int i = 0; i < kW; ++i) {
            if (ri[i] < 0) continue;
            if (bi < 0 || rv[i] > bv || (rv[i] == bv && ri[i] < bi)) {
                bv = rv[i];
                bi = ri[i];
            }
        }
        st_cross(a.cand + 2 * w, word1(tc_, __float_as_uint(bv)));
        st_cross(a.cand + 2 * w + 1, word1(tc_, (uint32_t)bi));
    }
    if (w != 0) return;
    float* cv = ar.att;   // 2 kG values
    const bool ok = poll_vec<1, kCross>(a, a.cand, 2 * kG, tc_, 6, [&](int i, uint32_t lo, uint32_t) {
        cv[i] = __uint_as_float(lo);
    });
    if (!__syncthreads_and(ok)) return;
    if ((tidx() >> 6) == 0) {
        float bv = -INFINITY;
        int bi = -1;
        for (int i = lane; i < kG; i += 64) {
            const int idx = (int)__float_as_uint(cv[2 * i + 1]);
            const float v = cv[2 * i];
            if (idx < 0) continue;
            if (bi < 0 || v > bv || (v == bv && idx < bi)) {
                bv = v;
                bi = idx;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            int32_t* scal = a.scal;
            scal[2] = bi;
            scal[0] = bi;
            scal[1] = pos + 1;
            const int32_t c = scal[3];
            scal[4 + c] = bi;
            scal[3] = c + 1;
        }
    }
    stamp(a, sh + 2);
}

// ---- host: instantiations, plan, launch ----------------------------------------------

using KFn = void (*)(Args);

struct Entry {
    int fq, fv, fv2, fo, fgu, fd, fd2, fh, hd;
    int H, slice_o, fxmax;   // K of stages A / D / head, C, E
    bool prefer;             // run this kernel even where the first one has an instantiation (measured faster)
    KFn fn;
};

#define P2(PREF, OPT, FQ, FV, FV2, FO, FGU, FD, FD2, FH, HD, H, SO, FX, LA, UA, NA, LC, UC, NC, LD, UD, ND, LE, UE, \
           NE, LH, UH, NH)                                                                                            \
    Entry {                                                                                                          \
        FQ, FV, FV2, FO, FGU, FD, FD2, FH, HD, H, SO, FX, PREF,                                                      \
            persist2_kernel<FQ, FV, FV2, FO, FGU, FD, FD2, FH, HD, LA, UA, NA, LC, UC, NC, LD, UD, ND, LE, UE, NE,  \
                            LH, UH, NH, OPT>                                                                         \
    }

constexpr int Q4 = FMT_Q4_K, Q6 = FMT_Q6_K, Q8 = FMT_Q8_0, F16 = FMT_F16;

// Shapes with an instantiation: the BASELINE widths and the test models.  The
// first argument says whether a shape runs here even where the first
// persistent kernel has an instantiation; the second holds the code options
// (kLate, kAsmDma).  Measured on MI355X (decode steps at a 1024-token
// context, ms; this kernel with its options / without options / the first
// kernel): 1.7B Q4_K 0.955 / 1.024 / 1.004, 0.6B Q8_0 0.741 / 0.765 / 0.976,
// 8B Q4_K 2.375 / 2.340 / 2.469 (kAsmDma 2.403; with the gammas requested
// early and the head's logits staged: both 2.256, none 2.303), Llama-3-8B widths
// 2.298 / 2.504 / 2.431.  The 1.7B Q4_K_M layout (1.072 / 1.071; no
// instantiation in the first kernel, 1.387 on the captured per-stage graph)
// takes the same options as the 1.7B.  The lm_head streams 4 rows per wave
// and buffer (8 rows: 63 us for the 1.7B's 255 MB, 4 rows: 54 us).
// Per stage (lanes per row, units per lane, passes): a wave's first task is
// requested one stage ahead; rows past it load in place.
constexpr int kBoth = kLate | kAsmDma;
const Entry kTable[] = {
    // Qwen3-1.7B (H 2048, F 6144, 16 / 8 heads): Q4_K with Q6_K v / down and an
    // untied Q6_K head; the same with v / down Q6_K or
    // Q4_K per layer and the tied FP16 head (the real Q4_K_M files)
    P2(true, kBoth, Q4, Q6, -1, Q4, Q4, Q6, -1, Q6, 128, 2048, 256, 768, 64, 1, 5, 8, 1, 2, 64, 1, 6, 8, 3, 2, 64, 1,
       4),
    P2(true, kBoth, Q4, Q6, Q4, Q4, Q4, Q6, Q4, F16, 128, 2048, 256, 768, 64, 1, 5, 8, 1, 2, 64, 1, 6, 8, 3, 2, 64, 1,
       4),
    // Qwen3-0.6B (H 1024, F 3072): Q8_0 with the tied FP16 head
    P2(true, kBoth, Q8, Q8, -1, Q8, Q8, Q8, -1, F16, 128, 1024, 256, 384, 32, 1, 2, 8, 1, 1, 32, 1, 2, 8, 2, 1, 32, 1,
       4),
    // Qwen3-8B (H 4096, F 12288, 32 / 8 heads): Q4_K, Q6_K head
    P2(true, kBoth, Q4, Q4, -1, Q4, Q4, Q4, -1, Q6, 128, 4096, 512, 1536, 64, 2, 4, 16, 1, 4, 64, 2, 2, 16, 3, 2, 64, 2,
       4),
    // Llama-3-8B widths (H 4096, F 14336): Q4_K with Q6_K v / down and head
    P2(true, kBoth, Q4, Q6, -1, Q4, Q4, Q6, -1, Q6, 128, 4096, 512, 1792, 64, 2, 4, 16, 1, 4, 64, 2, 2, 16, 4, 1, 64,
       2, 4),
    // test models: H 256 / head_dim 64 with F 2048 (Q4_K, Q6_K or Q4_K v / down, Q6_K head)
    P2(true, kBoth, Q4, Q6, Q4, Q4, Q4, Q6, Q4, Q6, 64, 256, 256, 256, 8, 1, 1, 8, 1, 1, 8, 1, 1, 8, 1, 1, 8, 1, 1),
    // H 512 / F 1024 / head_dim 64, Q8_0, tied FP16 head
    P2(true, kBoth, Q8, Q8, -1, Q8, Q8, Q8, -1, F16, 64, 512, 128, 128, 16, 1, 1, 4, 1, 1, 16, 1, 1, 4, 1, 1, 16, 1,
       1),
    // H 256 / F 6144 / head_dim 128, one KV head (Mistral-shaped, Q4_K / Q6_K)
    P2(true, kBoth, Q4, Q6, Q4, Q4, Q4, Q6, Q4, Q6, 128, 256, 512, 768, 8, 1, 1, 16, 1, 1, 8, 1, 1, 8, 3, 1, 8, 1, 1),
};

struct Plan {
    KFn fn = nullptr;
    int gpu = 0, nu = 0, aq = 0, ak = 0, av = 0, wq = 0, wk = 0, wv = 0, wqkv = 0, smax = 0, rec = 0, fblk = 0,
        wact = 0, wpart = 0;
    int qkv_stride = 0, rec_stride = 0, act_stride = 0, part_stride = 0, hup_stride = 0;
    size_t ctrl = 0, qkv = 0, recw = 0, act = 0, pwo = 0, pdn = 0, hupo = 0, hupd = 0, cand = 0, total = 0;
    size_t lds_dyn = 0;   // without the layer table
    bool prefer = false;
};

int type_elems(int t) { return t == BX_TYPE_Q8_0 ? 32 : (t == BX_TYPE_Q4_K || t == BX_TYPE_Q6_K ? 256 : 0); }
double row_bytes(int t, int K) { return (double)type_block_bytes(t) * K / (double)type_block_elems(t); }

int plan_of(const bx_decode_dims& d, Plan& o) {
    if (num_cus() != kG) return fail(BX_EUNSUPPORTED, "persist2: needs 256 CUs in 8 XCDs");
    const int hd = d.head_dim, H = d.hidden, F = d.intermediate;
    if (d.n_kv <= 0 || d.n_q % d.n_kv) return fail(BX_EINVAL, "persist2: bad head counts");
    const int Gq = d.n_q / d.n_kv;
    if (Gq != 1 && Gq != 2 && Gq != 4) return fail(BX_EUNSUPPORTED, "persist2: query heads per KV head not 1, 2 or 4");
    if (d.qkv_type_q != d.qkv_type_k || d.gate_type != d.up_type)
        return fail(BX_EUNSUPPORTED, "persist2: q/k or gate/up formats differ");
    const int blk_o = type_elems(d.o_type);
    if (blk_o == 0) return fail(BX_EUNSUPPORTED, "persist2: Wo format");
    int gpu = 0;
    for (int g = 1; g <= d.n_kv; ++g)
        if (d.n_kv % g == 0 && (g * Gq * hd) % blk_o == 0) {
            gpu = g;
            break;
        }
    if (gpu == 0 || d.n_kv / gpu > kX) return fail(BX_EUNSUPPORTED, "persist2: KV groups do not map onto 8 XCDs");
    const int nu = d.n_kv / gpu, smax = kR / gpu;
    const int vt[2] = {d.qkv_type_v, d.v_alt_type}, dt[2] = {d.down_type, d.down_alt_type};
    const int fblk = std::max(type_elems(d.down_type), type_elems(d.down_alt_type));
    if (fblk == 0 || F % fblk || H % 256 || H > 8 * kT * kGammaRounds)
        return fail(BX_EUNSUPPORTED, "persist2: widths");
    const int nbF = F / fblk, fxmax = (nbF + kX - 1) / kX * fblk;
    // Every XCD holds an FFN slice: its E stage then waits for all 32 of its
    // workgroups' D stages, which is what keeps an owner from overwriting an
    // h-update word (next layer) before a slow reader of its XCD has read it.
    if (nbF < kX) return fail(BX_EUNSUPPORTED, "persist2: FFN narrower than one block per XCD");
    const int slice_o = gpu * Gq * hd;
    const Entry* ent = nullptr;
    for (const Entry& e : kTable) {
        auto has = [](int t, int a, int b) { return t == 0 || t == a || (b >= 0 && t == b); };
        if (e.fq != d.qkv_type_q || e.fo != d.o_type || e.fgu != d.gate_type || e.fh != d.lm_type || e.hd != hd ||
            e.H != H || e.slice_o != slice_o || e.fxmax != fxmax)
            continue;
        if (!has(vt[0], e.fv, e.fv2) || !has(vt[1], e.fv, e.fv2) || !has(dt[0], e.fd, e.fd2) ||
            !has(dt[1], e.fd, e.fd2))
            continue;
        ent = &e;
        break;
    }
    if (!ent) return fail(BX_EUNSUPPORTED, "persist2: no instantiation for this format mix / width");
    o.fn = ent->fn;
    o.prefer = ent->prefer;
    o.gpu = gpu;
    o.nu = nu;
    o.smax = smax;
    o.fblk = fblk;
    // stage A: the 32 workgroups of a unit over its q, k and v rows, in
    // proportion to their bytes (every segment at least one)
    const int R[3] = {gpu * Gq * hd, gpu * hd, gpu * hd};
    const double vb = std::max(row_bytes(vt[0], H), vt[1] ? row_bytes(vt[1], H) : 0.0);
    const double b[3] = {R[0] * row_bytes(d.qkv_type_q, H), R[1] * row_bytes(d.qkv_type_k, H), R[2] * vb};
    int n[3];
    {
        const double tot = b[0] + b[1] + b[2];
        int sum = 0;
        for (int i = 0; i < 3; ++i) {
            n[i] = std::max(1, (int)(kR * b[i] / tot));
            sum += n[i];
        }
        while (sum < kR) {   // the next workgroup to the segment with the most bytes per workgroup
            int best = 0;
            for (int i = 1; i < 3; ++i)
                if (b[i] / n[i] > b[best] / n[best]) best = i;
            ++n[best];
            ++sum;
        }
        while (sum > kR) {
            int best = -1;
            for (int i = 0; i < 3; ++i)
                if (n[i] > 1 && (best < 0 || b[i] / (n[i] - 1) < b[best] / (n[best] - 1))) best = i;
            --n[best];
            --sum;
        }
    }
    o.aq = n[0];
    o.ak = n[1];
    o.av = n[2];
    o.wq = even(words3((R[0] + n[0] - 1) / n[0]));
    o.wk = even(words3((R[1] + n[1] - 1) / n[1]));
    o.wv = even(words3((R[2] + n[2] - 1) / n[2]));
    o.wqkv = o.aq * o.wq + o.ak * o.wk + o.av * o.wv;
    o.rec = even(words3(hd) + 2);
    o.wact = even(words3((fxmax + kR - 1) / kR));
    o.wpart = even(words3(H / kR));
    // rows a workgroup gathers before packing them (LDS rows[256])
    if ((R[0] + n[0] - 1) / n[0] > 256 || H / kR > 256 || (fxmax + kR - 1) / kR > 256)
        return fail(BX_EUNSUPPORTED, "persist2: too many rows per workgroup");
    // word buffers: per XCD regions on their own 256-byte lines
    auto up = [](size_t words) { return (words * 8 + 255) / 256 * 256 / 8; };
    o.qkv_stride = (int)up(o.wqkv);
    o.rec_stride = (int)up((size_t)gpu * smax * Gq * o.rec);
    o.act_stride = (int)up((size_t)kR * o.wact);
    o.part_stride = (int)up((size_t)H);
    o.hup_stride = (int)up((size_t)kR * o.wpart);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    o.ctrl = take(kCtrlBytes);
    o.qkv = take((size_t)kX * o.qkv_stride * 8);
    o.recw = take((size_t)kX * o.rec_stride * 8);
    o.act = take((size_t)kX * o.act_stride * 8);
    o.pwo = take((size_t)kX * o.part_stride * 8);
    o.pdn = take((size_t)kX * o.part_stride * 8);
    o.hupo = take((size_t)kX * o.hup_stride * 8);
    o.hupd = take((size_t)kX * o.hup_stride * 8);
    o.cand = take((size_t)2 * kG * 8);
    o.total = off;
    const int kmax = kmax_of(H, fxmax, slice_o);
    o.lds_dyn = arena_bytes(H, kmax, hd, gpu, Gq);
    // the combine's weights (heads x S) and the head's candidates live in the attention scratch
    if ((size_t)gpu * Gq * smax > att_floats(hd, gpu, Gq)) return fail(BX_EUNSUPPORTED, "persist2: scratch");
    // the head's FP16 logits of a workgroup's vocabulary rows are staged in the
    // attention tile (at least 2 kTile hd halves)
    if ((d.vocab + kG - 1) / kG > 2 * kTile * hd) return fail(BX_EUNSUPPORTED, "persist2: vocabulary too large");
    return BX_OK;
}

uint64_t* g_trace = nullptr;

__global__ void ws_init_kernel(uint32_t* ctrl, uint64_t* words, size_t nwords) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < kCtrlBytes / 4) ctrl[i] = 0u;
    for (size_t j = i; j < nwords; j += (size_t)gridDim.x * blockDim.x) words[j] = ~0ull;
}

// Which persistent kernel runs a shape: this one where its entry prefers it
// or the first kernel has no instantiation (per-layer attn_v / ffn_down
// formats, a tied FP16 head over Q4_K layers); BROLM_PERSIST_V1 /
// BROLM_PERSIST_V2 force one of the two.
bool use_p2(const bx_decode_dims* d, Plan& o) {
    static const bool v1 = std::getenv("BROLM_PERSIST_V1") != nullptr;
    static const bool v2 = std::getenv("BROLM_PERSIST_V2") != nullptr;
    if (v1 || !d) return false;
    if (plan_of(*d, o) != BX_OK) return false;
    if (v2 || o.prefer) return true;
    const std::string err = bx_last_error();
    const bool p1_ok = p1_ws_bytes(d) != 0;
    set_error(err);
    return !p1_ok;
}

}  // namespace
}  // namespace p2
}  // namespace bx

extern "C" size_t bx_persist_ws_bytes(const bx_decode_dims* d) {
    bx::p2::Plan o;
    if (bx::p2::use_p2(d, o)) return o.total;
    return bx::p1_ws_bytes(d);
}

extern "C" int bx_persist_ws_init(const bx_decode_dims* d, void* ws, void* stream) {
    bx::p2::Plan o;
    if (!bx::p2::use_p2(d, o)) return bx::p1_ws_init(d, ws, stream);
    if (!ws) return bx::fail(BX_EINVAL, "persist_ws_init: null workspace");
    unsigned char* base = static_cast<unsigned char*>(ws);
    hipLaunchKernelGGL(bx::p2::ws_init_kernel, dim3(256), dim3(256), 0, bx::as_stream(stream),
                       reinterpret_cast<uint32_t*>(base + o.ctrl), reinterpret_cast<uint64_t*>(base + o.qkv),
                       (o.total - o.qkv) / 8);
    if (hipGetLastError() != hipSuccess) return bx::fail(BX_ELAUNCH, "persist_ws_init: launch failed");
    return BX_OK;
}

extern "C" int bx_persist_step(const bx_decode_dims* d, int n_layers, const bx_decode_layer* layers_dev,
                               const uint16_t* embed, const uint16_t* final_norm, const void* lm_head,
                               const float* cos_tab, const float* sin_tab, int32_t* scal, uint16_t* logits,
                               void* ws, uint32_t epoch, void* stream) {
    using namespace bx::p2;
    Plan o;
    if (!use_p2(d, o))
        return bx::p1_step(d, n_layers, layers_dev, embed, final_norm, lm_head, cos_tab, sin_tab, scal, logits, ws,
                           epoch, stream);
    if (!layers_dev || !embed || !final_norm || !lm_head || !cos_tab || !sin_tab || !scal || !logits || !ws)
        return bx::fail(BX_EINVAL, "persist: null pointer");
    if (n_layers <= 0 || n_layers > 112) return bx::fail(BX_EINVAL, "persist: layer count");
    if (epoch == 0 || epoch >= 64) return bx::fail(BX_EINVAL, "persist: epoch out of range (1..63)");
    Args a{};
    a.H = d->hidden; a.F = d->intermediate; a.nq = d->n_q; a.nkv = d->n_kv; a.V = d->vocab; a.cap = d->cap;
    a.L = n_layers; a.eps = d->eps; a.qk_norm = d->no_qk_norm ? 0 : 1; a.epoch = epoch;
    a.gpu = o.gpu; a.nu = o.nu; a.aq = o.aq; a.ak = o.ak; a.av = o.av; a.wq = o.wq; a.wk = o.wk; a.wv = o.wv;
    a.wqkv = o.wqkv; a.smax = o.smax; a.rec = o.rec; a.fblk = o.fblk; a.wact = o.wact; a.wpart = o.wpart;
    a.layers = layers_dev; a.embed = embed; a.final_norm = final_norm; a.lm_head = lm_head;
    a.cos_t = cos_tab; a.sin_t = sin_tab; a.scal = scal; a.logits = logits;
    unsigned char* base = static_cast<unsigned char*>(ws);
    a.ctrl = reinterpret_cast<uint32_t*>(base + o.ctrl);
    a.qkv = reinterpret_cast<uint64_t*>(base + o.qkv);
    a.recw = reinterpret_cast<uint64_t*>(base + o.recw);
    a.act = reinterpret_cast<uint64_t*>(base + o.act);
    a.pwo = reinterpret_cast<uint64_t*>(base + o.pwo);
    a.pdn = reinterpret_cast<uint64_t*>(base + o.pdn);
    a.hupo = reinterpret_cast<uint64_t*>(base + o.hupo);
    a.hupd = reinterpret_cast<uint64_t*>(base + o.hupd);
    a.cand = reinterpret_cast<uint64_t*>(base + o.cand);
    a.qkv_stride = o.qkv_stride; a.rec_stride = o.rec_stride; a.act_stride = o.act_stride;
    a.part_stride = o.part_stride;
    a.hup_stride = o.hup_stride;
    a.trace = g_trace;
    const size_t lds = o.lds_dyn + table_bytes(n_layers);
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(o.fn)) != hipSuccess)
        return bx::fail(BX_ELAUNCH, "persist: kernel attributes");
    if (lds + attr.sharedSizeBytes > 160 * 1024) return bx::fail(BX_EUNSUPPORTED, "persist: LDS budget exceeded");
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(o.fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return bx::fail(BX_ELAUNCH, "persist: cannot raise the LDS limit");
    void* args[] = {&a};
    hipStream_t st = bx::as_stream(stream);
    // A plain launch of the grid after the occupancy check the cooperative
    // launch makes (one workgroup per CU, grid = CU count): on a device that
    // no other kernel holds the grid is resident at once, and the cooperative
    // launch's own cost (15-18 us a step on the GPU's timeline) is saved.
    // Every wait is bounded, so a grid that is not all resident (another
    // process's kernels on the CUs) ends with the abort flag set, and the
    // caller redoes the step another way.  BROLM_PERSIST_COOPERATIVE=1 takes
    // the cooperative launch instead, except under a profiler tool (rocprofv3
    // has ended processes whose kernels were launched cooperatively with a
    // segmentation fault in its exit path).
    static const bool plain = std::getenv("BROLM_PERSIST_COOPERATIVE") == nullptr || bx::profiler_attached();
    hipError_t e;
    if (plain) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(o.fn), kT, lds) !=
                hipSuccess ||
            per_cu < 1)
            return bx::fail(BX_ELAUNCH, "persist: workgroup does not fit on a CU");
        e = hipLaunchKernel(reinterpret_cast<const void*>(o.fn), dim3(kG), dim3(kT), args, lds, st);
    } else {
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(o.fn), dim3(kG), dim3(kT), args, (unsigned)lds,
                                       st);
    }
    if (e != hipSuccess) return bx::fail(BX_ELAUNCH, std::string("persist: launch failed: ") + hipGetErrorString(e));
    return BX_OK;
}

extern "C" int bx_persist_status(const void* ws, uint32_t* site) {
    if (!ws) return bx::fail(BX_EINVAL, "persist_status: null workspace");
    uint32_t c[2] = {0, 0};
    if (hipMemcpy(c, ws, sizeof(c), hipMemcpyDeviceToHost) != hipSuccess)
        return bx::fail(BX_ELAUNCH, "persist_status: copy failed");
    if (site) *site = c[1];
    return c[0] ? 1 : 0;
}

extern "C" int bx_persist_trace(uint64_t* buf_dev, int slots_per_wg) {
    if (buf_dev && slots_per_wg < bx::p2::kTraceSlots)
        return bx::fail(BX_EINVAL, "persist_trace: need 1024 slots per workgroup");
    bx::p2::g_trace = buf_dev;
    bx::p1_set_trace(buf_dev);
    return BX_OK;
}
