// Multi-sequence batched decode: the per-row forms of RoPE and the KV append
// (each of the M rows is the next token of its own sequence, at its own
// position, in its own slot of a slot-major KV arena), and the two fused with
// the q / k head RMSNorm into one launch.  The attention over
// each row's own keys is bx_attention_varlen_f16 (attention.hip).  These
// extend the single-sequence ops of src/detail/dense_decoder.cpp:585-607
// (rope_forward with one seq_offset, kv_cache_append at one cur_len).
#include "common.h"

namespace bx {
namespace {

// RoPE of one pair (2i, 2i+1) by the table angle (cos c, sin s), FP16 out.
// The arithmetic is fixed (one explicit fused multiply-add each, an FP32
// result, then FP16), so every kernel that rotates with this function rounds
// the same way; left to the compiler, which product it fuses, or a fusion
// with the FP16 conversion, may differ between kernels and move a result
// across an FP16 rounding boundary.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, uint16_t& y0, uint16_t& y1) {
    y0 = f2h(f32_fence(__builtin_fmaf(x0, c, -f32_fence(x1 * s))));
    y1 = f2h(f32_fence(__builtin_fmaf(x0, s, f32_fence(x1 * c))));
}

// Row r rotates at position pos[r]; rows whose position is outside the table
// are left unwritten (the host validates positions before the launch).
__global__ void rope_rows_kernel(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int rows, int hd,
                                 int n_heads, const int32_t* __restrict__ pos, int tab_rows,
                                 const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * n_heads * half) return;
    const int p = (int)(i % half);
    const int64_t rh = i / half;
    const int r = (int)(rh / n_heads);
    const int ps = pos[r];
    if (ps < 0 || ps >= tab_rows) return;
    const int64_t off = rh * hd + 2 * p;
    const float c = cos_t[(int64_t)ps * half + p], s = sin_t[(int64_t)ps * half + p];
    uint16_t y0, y1;
    rope_pair(h2f(X[off]), h2f(X[off + 1]), c, s, y0, y1);
    Y[off] = y0;
    Y[off + 1] = y1;
}

// Row r of k / v goes to cache row dst[r] (slot * capacity + position);
// rows outside [0, cache_rows) are skipped.
__global__ void kv_rows_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int rows, int cols,
                               const int64_t* __restrict__ dst, int64_t cache_rows, uint16_t* __restrict__ Kc,
                               uint16_t* __restrict__ Vc) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i % cols);
    const int64_t d = dst[r];
    if (d < 0 || d >= cache_rows) return;
    Kc[d * cols + c] = k[i];
    Vc[d * cols + c] = v[i];
}

// The per-head stage of a batched step in one launch: for row r and head h
// (q heads, then k heads), the head RMSNorm (when a gain is given), RoPE at
// pos[r], and the k row (with its v row) written to cache row dst[r].  One
// wavefront per (row, head); lane l holds elements l, l + 64, ... of the head,
// as the one-wavefront rms_norm_kernel does, so the sum of squares, the FP16
// normed values and the rotation round exactly as the separate launches of
// rms_norm, rope_rows and kv_append_rows.  A pair's partner element is in the
// neighbouring lane.
// One head (64 EPL elements, lane l holding elements l, l + 64, ...) of a raw
// projection row: RMSNorm with gain (when given), FP16, RoPE by the table row
// ps (identity when rot is false), FP16.  y[i] is element lane + 64 i.  The
// loads (load) and the arithmetic (apply) are apart, so a caller can request
// the inputs of several heads before it waits for any.
template <int EPL>
struct NormRopeLane {
    uint32_t x[EPL], gm[EPL];
    float c[EPL], sn[EPL];
    // Every load unconditional, so no branch join waits for one: without a
    // gain the row itself is read in its place, off the table (rot false) its
    // row 0 (launchers require a table of at least one row); apply takes the
    // flags.
    __device__ __forceinline__ void load(const uint16_t* src, const uint16_t* gain, int ps, bool rot,
                                         const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
        constexpr int half = 32 * EPL;
        const int lane = threadIdx.x & 63;
        const uint16_t* gp = gain ? gain : src;
        const int64_t row = rot ? ps : 0;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            x[i] = src[e];
            gm[i] = gp[e];
            c[i] = cos_t[row * half + (e >> 1)];
            sn[i] = sin_t[row * half + (e >> 1)];
        }
    }
    __device__ __forceinline__ void apply(bool gain, bool rot, float eps, uint16_t (&y)[EPL]) const {
        constexpr int HD = 64 * EPL;
        const int lane = threadIdx.x & 63;
        float xf[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) xf[i] = h2f((uint16_t)x[i]);
        if (gain) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < EPL; ++i) ss += xf[i] * xf[i];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
            for (int i = 0; i < EPL; ++i) xf[i] = h2f(norm_f16(xf[i], inv, h2f((uint16_t)gm[i])));
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            const float other = __shfl_xor(xf[i], 1, 64);
            const float cc = rot ? c[i] : 1.f, ss = rot ? sn[i] : 0.f;
            uint16_t y0, y1;
            if (e & 1) rope_pair(other, xf[i], cc, ss, y0, y1);
            else rope_pair(xf[i], other, cc, ss, y0, y1);
            y[i] = (e & 1) ? y1 : y0;
        }
    }
};

template <int EPL>
__device__ __forceinline__ void norm_rope_lane(const uint16_t* src, const uint16_t* gain, float eps, int ps, bool rot,
                                               const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                               uint16_t (&y)[EPL]) {
    NormRopeLane<EPL> n;
    n.load(src, gain, ps, rot, cos_t, sin_t);
    n.apply(gain != nullptr, rot, eps, y);
}

template <int EPL>
__global__ __launch_bounds__(256) void qk_rope_kv_rows_kernel(
    const uint16_t* q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int rows, int n_q, int n_kv, const uint16_t* __restrict__ q_gain, const uint16_t* __restrict__ k_gain, float eps,
    const int32_t* __restrict__ pos, int tab_rows, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int64_t* __restrict__ dst, int64_t cache_rows, uint16_t* __restrict__ Kc, uint16_t* __restrict__ Vc,
    uint16_t* q_out) {
    constexpr int HD = 64 * EPL;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int heads = n_q + n_kv;
    if (item >= rows * heads) return;
    const int lane = threadIdx.x & 63;
    const int r = item / heads, h = item - r * heads;
    const bool is_q = h < n_q;
    const int hk = h - n_q;
    const uint16_t* src = is_q ? q + ((int64_t)r * n_q + h) * HD : k + ((int64_t)r * n_kv + hk) * HD;
    const int ps = pos[r];
    const bool rot = ps >= 0 && ps < tab_rows;
    uint16_t y[EPL];
    norm_rope_lane<EPL>(src, is_q ? q_gain : k_gain, eps, ps, rot, cos_t, sin_t, y);
    if (is_q) {
        if (!rot) return;
        uint16_t* o = q_out + ((int64_t)r * n_q + h) * HD;
#pragma unroll
        for (int i = 0; i < EPL; ++i) o[lane + 64 * i] = y[i];
        return;
    }
    const int64_t d = dst[r];
    if (!rot || d < 0 || d >= cache_rows) return;
    const int64_t width = (int64_t)n_kv * HD;
    const uint16_t* vs = v + (int64_t)r * width + (int64_t)hk * HD;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        Kc[d * width + (int64_t)hk * HD + e] = y[i];
        Vc[d * width + (int64_t)hk * HD + e] = vs[e];
    }
}

// ---- batched attention with the per-head stage fused ------------------------
//
// One launch per layer of a batched step: workgroup (split s, KV group g, row
// r) takes keys [s kps, s kps + kps) of row r's own sequence (cache rows
// base[r] + j, its new key at j = lens[r] - 1).  Its prologue normalises and
// rotates the group's q heads (norm_rope_lane, the arithmetic of the separate
// q / k stage), and the split that holds the new key does the same for the new
// k row and writes k and v to the cache (and into its LDS tile in place of the
// stale row).  Key tiles are copied to LDS (K in 16-byte chunks XOR-swizzled
// by the key, so lanes reading consecutive keys hit distinct banks); each
// wavefront then works alone on a key part x head: one lane per key for the
// scores (v_dot2 on FP16 q and k), an online softmax in registers, P.V with
// the probabilities broadcast by readlane and EPL head dims per lane.  The key
// parts of a head are merged in LDS; the (o, m, l) record of each (split,
// head) goes out by device-scope stores, and the workgroup of a (row, group)
// that finishes last merges its S records in split order (the result does not
// depend on arrival order), writes the FP16 output and returns the counter to
// zero.
template <int HD>
struct BaShape {
    static constexpr int TK = 8192 / HD;   // keys per LDS tile (two tiles of K and V: 64 KB)
    static constexpr int CPK = HD / 8;     // 16-byte chunks per key row
    static constexpr int EPL = HD / 64;    // head elements (and output dims) per lane
    static constexpr int INST = TK * CPK / 64;   // copy instructions of a tile (K or V), a multiple of 4
};

struct BatchAttnArgs {
    const uint16_t* q;     // rows x n_q HD, raw projections
    const uint16_t* k;     // rows x n_kv HD
    const uint16_t* v;
    const uint16_t* q_gain;   // null: no head norm
    const uint16_t* k_gain;
    float eps;
    const int32_t* lens;   // keys of row r with its new one (position lens[r] - 1)
    const int64_t* base;   // cache row of key 0 of row r
    const float* cos_t;
    const float* sin_t;
    int tab_rows;
    uint16_t* Kc;
    uint16_t* Vc;
    int64_t cache_rows;
    int n_q, n_kv, S, kps, P, HPW;
    float* recs;       // (row, group) x S x G records of HD + 2 floats
    uint64_t* cnt;     // rows x n_kv counter words (tagged_arrive), zero between launches
    uint32_t tag;      // this launch's tag (nonzero)
    uint16_t* out;     // rows x n_q HD
};

constexpr int kBaSc1 = 16;   // cache policy of the record stores and loads: sc1, device scope

template <int HD>
__device__ __forceinline__ void ba_dma(const void* src, uint16_t* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(256) void batch_attn_kernel(BatchAttnArgs a) {
    using SH = BaShape<HD>;
    constexpr int TK = SH::TK, CPK = SH::CPK, EPL = SH::EPL;
    extern __shared__ __align__(16) uint16_t ba_lds[];
    // the roped q heads and the new k / v rows apart from the tiles: writes
    // there need not wait for the tile copies in flight
    __shared__ __align__(16) uint16_t ba_qkv[10 * HD];
    __shared__ uint32_t last;
    uint16_t* tiles = ba_lds;          // two buffers of K (TK x HD, swizzled chunks) then V (TK x HD)
    uint16_t* qs = ba_qkv;             // 8 x HD roped q heads
    uint16_t* kn = qs + 8 * HD;        // the new key row
    uint16_t* vn = kn + HD;            // the new value row
    const int s = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
    const int G = a.n_q / a.n_kv, P = a.P, HPW = a.HPW, T = a.S;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int len = a.lens[r], pnew = len - 1;
    const int kb = s * a.kps, ke = min(len, kb + a.kps);
    const bool has_cur = kb <= pnew && pnew < ke;
    const int64_t kvd = (int64_t)a.n_kv * HD;
    const int64_t row0 = a.base[r];
    const bool rot = pnew >= 0 && pnew < a.tab_rows;
    const uint16_t* Kg = a.Kc + row0 * kvd + (int64_t)g * HD;
    const uint16_t* Vg = a.Vc + row0 * kvd + (int64_t)g * HD;
    // tile copy of keys [c0, c0 + nk) into buffer b; slots past nk repeat key
    // nk - 1 (in bounds).  A wavefront issues the same copies whatever nk, so
    // the waits for the loads requested before them count exactly.
    auto copy_tile = [&](int b, int c0, int nk) {
        uint16_t* kt = tiles + 2 * b * TK * HD;
        uint16_t* vt = kt + TK * HD;
        static_assert(SH::INST % 4 == 0, "copy instructions per wavefront");
#pragma unroll
        for (int k4 = 0; k4 < SH::INST / 4; ++k4) {
            const int i = wave + 4 * k4;
            const int slot = 64 * i + lane;
            int j = slot / CPK;
            const int pc = slot % CPK;
            if (j >= nk) j = nk - 1;
            const int64_t rowo = (int64_t)(c0 + j) * kvd;
            ba_dma<HD>(Kg + rowo + 8 * (pc ^ (j & (CPK - 1))), kt + 512 * i);
            ba_dma<HD>(Vg + rowo + 8 * pc, vt + 512 * i);
        }
    };
    // ---- prologue: the inputs of the group's q heads (at most two per
    // wavefront) and, in the split holding the new key, of its k and v rows
    // are requested first and the first tile's copy right behind them (loads
    // complete in issue order); then the roped q heads and the new k / v rows
    // (unconditional loads at clamped heads, so no branch join waits for
    // them; only the heads that exist are used)
    NormRopeLane<EPL> qin[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int hh = min(wave + 4 * i, G - 1);
        qin[i].load(a.q + ((int64_t)r * a.n_q + g * G + hh) * HD, a.q_gain, pnew, rot, a.cos_t, a.sin_t);
    }
    const bool cur_wave = has_cur && wave == 3;
    NormRopeLane<EPL> kin;
    uint32_t vin[EPL];
    kin.load(a.k + (int64_t)r * kvd + (int64_t)g * HD, a.k_gain, pnew, rot, a.cos_t, a.sin_t);
    {
        const uint16_t* vs = a.v + (int64_t)r * kvd + (int64_t)g * HD;
#pragma unroll
        for (int i = 0; i < EPL; ++i) vin[i] = vs[lane + 64 * i];
    }
    // the first tile lands while the prologue runs; an empty split copies a
    // row of its sequence it does not read, so every wavefront issues the
    // same copies (the waits for the prologue's loads then count exactly)
    copy_tile(0, max(0, min(kb, len - 1)), max(1, min(TK, ke - kb)));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int hh = wave + 4 * i;
        if (hh < G) {
            uint16_t y[EPL];
            qin[i].apply(a.q_gain != nullptr, rot, a.eps, y);
#pragma unroll
            for (int e = 0; e < EPL; ++e) qs[hh * HD + lane + 64 * e] = y[e];
        }
    }
    if (cur_wave) {
        uint16_t y[EPL];
        kin.apply(a.k_gain != nullptr, rot, a.eps, y);
        const int64_t d = row0 + pnew;
        const bool write = rot && d >= 0 && d < a.cache_rows;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            kn[e] = y[i];
            vn[e] = (uint16_t)vin[i];
            if (write) {
                a.Kc[d * kvd + (int64_t)g * HD + e] = y[i];
                a.Vc[d * kvd + (int64_t)g * HD + e] = (uint16_t)vin[i];
            }
        }
    }

    // ---- key tiles: each wavefront a key part x HPW heads, its own softmax
    const int part = wave % P, h0 = (wave / P) * HPW;
    const float scale = 1.0f / sqrtf((float)HD);
    float m_run[2], l_run[2], o[2][EPL];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        m_run[hh] = -INFINITY;
        l_run[hh] = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) o[hh][i] = 0.f;
    }
    for (int c0 = kb, it = 0; c0 < ke; c0 += TK, ++it) {
        const int nk = min(TK, ke - c0);
        uint16_t* kt = tiles + 2 * (it & 1) * TK * HD;
        uint16_t* vt = kt + TK * HD;
        // this tile landed, and every wave is done with the other buffer:
        // the next tile's copy goes there and overlaps this tile's math
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (c0 + TK < ke) copy_tile((it & 1) ^ 1, c0 + TK, min(TK, ke - c0 - TK));
        if (has_cur && pnew >= c0 && pnew < c0 + nk) {
            const int jc = pnew - c0;
            for (int d8 = threadIdx.x; d8 < CPK; d8 += 256) {
                *reinterpret_cast<u4v*>(kt + jc * HD + 8 * (d8 ^ (jc & (CPK - 1)))) =
                    *reinterpret_cast<const u4v*>(kn + 8 * d8);
                *reinterpret_cast<u4v*>(vt + jc * HD + 8 * d8) = *reinterpret_cast<const u4v*>(vn + 8 * d8);
            }
            __syncthreads();
        }
        const int kpp = (nk + P - 1) / P;
        const int jb = min(nk, part * kpp), nkw = min(nk, jb + kpp) - jb;   // <= 128 keys: two per lane at most
        if (nkw > 0) {
            // unrolled over the (at most two) heads of the wave: the running
            // state stays in registers with fixed indices
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = h0 + hh;
                if (hh >= HPW || h >= G) continue;   // uniform
                const uint16_t* qh = qs + h * HD;
                float sv[2];
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    const int t = lane + 64 * hb;
                    sv[hb] = -INFINITY;
                    if (64 * hb < nkw) {   // uniform
                        const int jr = jb + (t < nkw ? t : nkw - 1);
                        const uint16_t* kr = kt + jr * HD;
                        float acc = 0.f, acc2 = 0.f;
#pragma unroll
                        for (int d0 = 0; d0 < CPK; d0 += 8) {
                            u4v kk[8], qv[8];
#pragma unroll
                            for (int c = 0; c < 8; ++c) {
                                kk[c] = *reinterpret_cast<const u4v*>(kr + 8 * ((d0 + c) ^ (jr & (CPK - 1))));
                                qv[c] = *reinterpret_cast<const u4v*>(qh + 8 * (d0 + c));
                            }
                            asm volatile("" ::: "memory");
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
                const float mt = wave_max(fmaxf(sv[0], sv[1]));
                const float mn = fmaxf(m_run[hh], mt);
                const float al = m_run[hh] == -INFINITY ? 0.f : __expf(m_run[hh] - mn);
                float pv[2];
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) pv[hb] = lane + 64 * hb < nkw ? __expf(sv[hb] - mn) : 0.f;
                l_run[hh] = l_run[hh] * al + wave_sum(pv[0] + pv[1]);
                m_run[hh] = mn;
#pragma unroll
                for (int i = 0; i < EPL; ++i) o[hh][i] *= al;
                // P.V: lane holds dims EPL lane .. EPL lane + EPL - 1
                const uint16_t* vcol = vt + jb * HD + EPL * lane;
                for (int t0 = 0; t0 < nkw; t0 += 8) {
                    uint16_t vv[8][EPL];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int t = min(t0 + u, nkw - 1);
#pragma unroll
                        for (int i = 0; i < EPL; ++i) vv[u][i] = vcol[t * HD + i];
                    }
                    asm volatile("" ::: "memory");
                    // keys past nkw (up to the next multiple of 8, below 128)
                    // have p = 0 and a clamped, finite value row
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int t = t0 + u;   // uniform
                        const float pt = __builtin_bit_cast(
                            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t < 64 ? pv[0] : pv[1]), t & 63));
#pragma unroll
                        for (int i = 0; i < EPL; ++i) o[hh][i] += pt * h2f(vv[u][i]);
                    }
                }
            }
        }
    }
    // an empty split left its one tile copy in flight: it lands before the
    // merge area (the tile buffers) is written
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();   // all waves are done with the tiles (the merge area reuses them)

    // ---- the P key parts of each head merged in LDS (the tile area is free
    // after the last barrier), then one record (o, m, l) per (split, head)
    const int rec = HD + 2;
    float* pl = reinterpret_cast<float*>(ba_lds);   // P x G records
    if (P > 1) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = h0 + hh;
            if (hh >= HPW || h >= G) continue;
            float* pr = pl + (part * G + h) * rec;
#pragma unroll
            for (int i = 0; i < EPL; ++i) pr[EPL * lane + i] = o[hh][i];
            if (lane == 0) {
                pr[HD] = m_run[hh];
                pr[HD + 1] = l_run[hh];
            }
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = h0 + hh;
                if (hh >= HPW || h >= G) continue;
                float mm = -INFINITY;
                for (int q = 0; q < P; ++q) mm = fmaxf(mm, pl[(q * G + h) * rec + HD]);
                float ll = 0.f, oo[EPL];
#pragma unroll
                for (int i = 0; i < EPL; ++i) oo[i] = 0.f;
                for (int q = 0; q < P; ++q) {
                    const float* pr = pl + (q * G + h) * rec;
                    const float w = pr[HD] == -INFINITY ? 0.f : __expf(pr[HD] - mm);
                    ll += w * pr[HD + 1];
#pragma unroll
                    for (int i = 0; i < EPL; ++i) oo[i] += w * pr[EPL * lane + i];
                }
                m_run[hh] = mm;
                l_run[hh] = ll;
#pragma unroll
                for (int i = 0; i < EPL; ++i) o[hh][i] = oo[i];
            }
        }
    }
    float* grp = a.recs + ((int64_t)r * a.n_kv + g) * (int64_t)T * G * rec;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(grp, 0, 0x7fffffff, 0x00020000);
    if (part == 0) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = h0 + hh;
            if (hh >= HPW || h >= G) continue;
            const int ro = (s * G + h) * rec;   // record offset, floats
#pragma unroll
            for (int i = 0; i < EPL; ++i)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o[hh][i]), rs,
                                                      4 * (ro + EPL * lane + i), 0, kBaSc1);
            if (lane == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, m_run[hh]), rs, 4 * (ro + HD), 0,
                                                      kBaSc1);
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, l_run[hh]), rs, 4 * (ro + HD + 1),
                                                      0, kBaSc1);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // the split's arrival count (tagged_arrive: a word left by a launch that
    // did not finish is not counted; the last arrival clears the word)
    uint64_t* cn = a.cnt + (int64_t)r * a.n_kv + g;
    if (threadIdx.x == 0) last = tagged_arrive(cn, a.tag) == (uint32_t)a.S ? 1u : 0u;
    __syncthreads();
    if (!last) return;

    // ---- merge of the group's S records per head, in split order: m and l of
    // every record in one pass (lane t <-> record t), the weights broadcast by
    // readlane, the o rows requested sixteen records at a time
    for (int h = wave; h < G; h += 4) {
        float mt[4], lt[4], wt[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int t = min(lane + 64 * k, T - 1);
            mt[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * ((t * G + h) * rec + HD), 0,
                                                                                     kBaSc1));
            lt[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  rs, 4 * ((t * G + h) * rec + HD + 1), 0, kBaSc1));
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (lane + 64 * k < T) mloc = fmaxf(mloc, mt[k]);
        const float M = wave_max(mloc);
        float lloc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = lane + 64 * k < T && mt[k] != -INFINITY;
            wt[k] = in ? __expf(mt[k] - M) : 0.f;
            lloc += wt[k] * (in ? lt[k] : 0.f);
        }
        const float L = wave_sum(lloc);
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        float acc[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) acc[i] = 0.f;
        for (int t0 = 0; t0 < T; t0 += 16) {
            float ov[16][EPL];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int t = min(t0 + u, T - 1);
#pragma unroll
                for (int i = 0; i < EPL; ++i)
                    ov[u][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                             rs, 4 * ((t * G + h) * rec + EPL * lane + i), 0, kBaSc1));
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int t = t0 + u;   // uniform
                if (t < T) {
                    const float w = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt[t >> 6]), t & 63));
#pragma unroll
                    for (int i = 0; i < EPL; ++i) acc[i] += w * ov[u][i];
                }
            }
        }
        uint16_t* op = a.out + ((int64_t)r * a.n_q + g * G + h) * HD + EPL * lane;
#pragma unroll
        for (int i = 0; i < EPL; ++i) op[i] = f2h(acc[i] * inv);
    }
    if (threadIdx.x == 0) __hip_atomic_store(cn, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split plan of the batched attention: about two workgroups per CU over all
// (row, group) pairs, at least 64 keys a split; P key parts per tile and HPW
// heads per wavefront from the group size G (four wavefronts).
struct BaPlan {
    int S, kps, P, HPW;
};
inline BaPlan ba_plan(int rows, int n_q, int n_kv, int max_len) {
    BaPlan p;
    const int G = n_q / n_kv;
    p.P = G >= 4 ? 1 : 4 / G;
    p.HPW = G > 4 ? (G + 3) / 4 : 1;
    int S = (2 * num_cus()) / max(1, rows * n_kv);
    S = max(1, min(min(S, (max_len + 63) / 64), 256));   // the merge takes at most 256 records
    p.kps = ((max_len + S - 1) / S + 15) / 16 * 16;
    p.S = (max_len + p.kps - 1) / p.kps;
    return p;
}
inline size_t ba_lds_bytes(int) { return (size_t)4 * 8192 * 2; }

inline unsigned blocks_of(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

int bx_rope_rows_f16(const uint16_t* X, uint16_t* Y, int rows, int hd, int n_heads, const int32_t* pos_dev,
                     const float* cos_tab, const float* sin_tab, int tab_rows, void* stream) {
    if (!X || !Y || !pos_dev || !cos_tab || !sin_tab || rows <= 0 || hd <= 0 || hd % 2 || n_heads <= 0 ||
        tab_rows <= 0)
        return fail(BX_EINVAL, "rope_rows: bad arguments");
    const int64_t n = (int64_t)rows * n_heads * (hd / 2);
    rope_rows_kernel<<<blocks_of(n, 256), 256, 0, as_stream(stream)>>>(X, Y, rows, hd, n_heads, pos_dev, tab_rows,
                                                                        cos_tab, sin_tab);
    return launch_check("rope_rows");
}

int bx_kv_append_rows_f16(const uint16_t* k, const uint16_t* v, int rows, int cols, const int64_t* dst_rows_dev,
                          uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, void* stream) {
    if (!k || !v || !dst_rows_dev || !Kc || !Vc || rows <= 0 || cols <= 0 || cache_rows <= 0)
        return fail(BX_EINVAL, "kv_append_rows: bad arguments");
    kv_rows_kernel<<<blocks_of((int64_t)rows * cols, 256), 256, 0, as_stream(stream)>>>(k, v, rows, cols,
                                                                                          dst_rows_dev, cache_rows,
                                                                                          Kc, Vc);
    return launch_check("kv_append_rows");
}

size_t bx_batch_attention_workspace_bytes(int rows, int n_q, int n_kv, int hd, int max_len) {
    if (rows <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv || hd <= 0 || max_len <= 0) return 0;
    const BaPlan p = ba_plan(rows, n_q, n_kv, max_len);
    const size_t cnt = ((size_t)rows * n_kv * 8 + 255) / 256 * 256;
    return cnt + (size_t)rows * n_q * p.S * (hd + 2) * sizeof(float);
}

int bx_batch_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int rows, int hd, int n_q,
                           int n_kv, const uint16_t* q_gain, const uint16_t* k_gain, float eps, const int32_t* lens_dev,
                           const int64_t* base_rows_dev, int max_len, const float* cos_tab, const float* sin_tab,
                           int tab_rows, uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, uint16_t* out,
                           void* workspace, void* stream) {
    if (!q || !k || !v || !lens_dev || !base_rows_dev || !cos_tab || !sin_tab || !Kc || !Vc || !out || !workspace ||
        rows <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv || max_len <= 0 || tab_rows <= 0 || cache_rows <= 0 ||
        (q_gain == nullptr) != (k_gain == nullptr))
        return fail(BX_EINVAL, "batch_attention: bad arguments");
    if (n_q / n_kv > 8) return fail(BX_EUNSUPPORTED, "batch_attention: at most 8 query heads per KV head");
    const BaPlan p = ba_plan(rows, n_q, n_kv, max_len);
    const size_t cnt = ((size_t)rows * n_kv * 8 + 255) / 256 * 256;
    if ((size_t)rows * n_q * p.S * (hd + 2) * sizeof(float) >= (size_t)1 << 31)
        return fail(BX_EUNSUPPORTED, "batch_attention: records beyond 2 GiB");
    BatchAttnArgs a{};
    a.q = q; a.k = k; a.v = v;
    a.q_gain = q_gain; a.k_gain = k_gain; a.eps = eps;
    a.lens = lens_dev; a.base = base_rows_dev;
    a.cos_t = cos_tab; a.sin_t = sin_tab; a.tab_rows = tab_rows;
    a.Kc = Kc; a.Vc = Vc; a.cache_rows = cache_rows;
    a.n_q = n_q; a.n_kv = n_kv; a.S = p.S; a.kps = p.kps; a.P = p.P; a.HPW = p.HPW;
    a.cnt = static_cast<uint64_t*>(workspace);
    a.tag = next_launch_tag();
    a.recs = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + cnt);
    a.out = out;
    const dim3 grid((unsigned)p.S, (unsigned)n_kv, (unsigned)rows);
    const size_t lds = ba_lds_bytes(hd);
    hipStream_t st = as_stream(stream);
    auto launch = [&](const void* fn, auto kern) -> int {
        static bool attr_done[3] = {false, false, false};
        const int slot = hd == 64 ? 0 : hd == 128 ? 1 : 2;
        if (!attr_done[slot] && lds > 64 * 1024) {
            if (int rc = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                   "batch_attention: LDS attribute"))
                return rc;
            attr_done[slot] = true;
        }
        kern<<<grid, 256, lds, st>>>(a);
        return launch_check("batch_attention");
    };
    switch (hd) {
        case 64: return launch(reinterpret_cast<const void*>(&batch_attn_kernel<64>), batch_attn_kernel<64>);
        case 128: return launch(reinterpret_cast<const void*>(&batch_attn_kernel<128>), batch_attn_kernel<128>);
        case 256: return launch(reinterpret_cast<const void*>(&batch_attn_kernel<256>), batch_attn_kernel<256>);
        default: return fail(BX_EUNSUPPORTED, "batch_attention: head_dim must be 64, 128 or 256");
    }
}

int bx_qk_rope_kv_rows_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int rows, int hd, int n_q,
                           int n_kv, const uint16_t* q_gain, const uint16_t* k_gain, float eps, const int32_t* pos_dev,
                           const float* cos_tab, const float* sin_tab, int tab_rows, const int64_t* dst_rows_dev,
                           uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, uint16_t* q_out, void* stream) {
    if (!q || !k || !v || !pos_dev || !cos_tab || !sin_tab || !dst_rows_dev || !Kc || !Vc || !q_out || rows <= 0 ||
        n_q <= 0 || n_kv <= 0 || tab_rows <= 0 || cache_rows <= 0 || (q_gain == nullptr) != (k_gain == nullptr))
        return fail(BX_EINVAL, "qk_rope_kv_rows: bad arguments");
    const unsigned grid = blocks_of((int64_t)rows * (n_q + n_kv), 4);
    hipStream_t st = as_stream(stream);
    switch (hd) {
        case 64:
            qk_rope_kv_rows_kernel<1><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        case 128:
            qk_rope_kv_rows_kernel<2><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        case 256:
            qk_rope_kv_rows_kernel<4><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        default:
            return fail(BX_EUNSUPPORTED, "qk_rope_kv_rows: head_dim must be 64, 128 or 256");
    }
    return launch_check("qk_rope_kv_rows");
}

}  // extern "C"
