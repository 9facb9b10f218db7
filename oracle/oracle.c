/*
 * oracle.c — CPU restatement of brolm's quantized Qwen3 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (checker for the HIP path; never part of the
 * product).  See oracle.h for what each part restates and where it is cited.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   fp16/bf16 conversions  - exhaustive over all 65536 fp16 codes (round trip)
 *                            and numpy's float16 cast on random + edge floats.
 *   dequant Q8_0/Q4_K/Q6_K - blocks built by an independent encoder from chosen
 *                            integer fields, closed form y = d*sc*q - dmin*m;
 *                            brute force of get_scale_min_k4 over all indices;
 *                            committed golden block vectors.
 *   GGUF reader            - files written by the product writer and by a
 *                            hand-assembled byte string in the tests.
 *   ops                    - closed forms / invariants (norm scale invariance,
 *                            rotation norm preservation + relative-position
 *                            property, one-hot attention, GQA map).
 *   whole decoder          - Hugging Face transformers Qwen3ForCausalLM in
 *                            float64 on the same dequantized (unpermuted)
 *                            weights: an independent implementation using
 *                            rotate_half RoPE, which checks the row permute too.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                         */
/* ------------------------------------------------------------------------- */

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    uint32_t E = ax >> 23;
    if (E < 113) { /* |f| < 2^-14: fp16 subnormal (or zero), unit 2^-24 */
        uint32_t mfull = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)E;
        if (E == 0 || shift > 24) return (uint16_t)sign;
        uint32_t q = mfull >> shift;
        uint32_t rem = mfull & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = ((E - 127 + 15) << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

void or_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}
void or_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------- */
/* block formats                                                              */
/* ------------------------------------------------------------------------- */

int64_t or_type_block_elems(int type) {
    switch (type) {
        case OR_T_Q8_0: return 32;
        case OR_T_Q4_K: case OR_T_Q6_K: return 256;
        case OR_T_F32: case OR_T_F16: case OR_T_BF16: return 1;
        default: return 0;
    }
}
int64_t or_type_block_bytes(int type) {
    switch (type) {
        case OR_T_Q8_0: return 34;
        case OR_T_Q4_K: return 144;
        case OR_T_Q6_K: return 210;
        case OR_T_F32: return 4;
        case OR_T_F16: case OR_T_BF16: return 2;
        default: return 0;
    }
}
int64_t or_row_bytes(int type, int64_t cols) {
    int64_t be = or_type_block_elems(type);
    if (be <= 0 || cols % be) return -1;
    return cols / be * or_type_block_bytes(type);
}

/* Q4_K super-block scales: 8 sub-blocks x (6-bit scale, 6-bit min) in 12 bytes.
 * Sub-blocks 0-3 keep their low 6 bits in bytes 0-3 (scale) and 4-7 (min);
 * sub-blocks 4-7 keep their low 4 bits in the nibbles of bytes 8-11 and their
 * high 2 bits in the top bits of bytes 0-7 (ggml get_scale_min_k4). */
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static void dq_q8_0_block(const uint8_t* b, float* y) {
    uint16_t dh;
    memcpy(&dh, b, 2);
    const float d = or_f16_to_f32(dh);
    const int8_t* qs = (const int8_t*)(b + 2);
    for (int i = 0; i < 32; ++i) y[i] = d * (float)qs[i];
}

/* block_q4_K: fp16 d, fp16 dmin, u8 scales[12], u8 qs[128].
 * qs chunk c (32 bytes) holds sub-block 2c in its low nibbles and 2c+1 in its
 * high nibbles; y = (d*sc)*q - (dmin*m). */
static void dq_q4_k_block(const uint8_t* b, float* y) {
    uint16_t dh, mh;
    memcpy(&dh, b, 2);
    memcpy(&mh, b + 2, 2);
    const float d = or_f16_to_f32(dh);
    const float dmin = or_f16_to_f32(mh);
    const uint8_t* scales = b + 4;
    const uint8_t* qs = b + 16;
    for (int c = 0; c < 4; ++c) {
        uint8_t sc0, m0, sc1, m1;
        or_get_scale_min_k4(2 * c, scales, &sc0, &m0);
        or_get_scale_min_k4(2 * c + 1, scales, &sc1, &m1);
        const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            y[64 * c + l] = d0 * (float)(qs[32 * c + l] & 0x0f) - mm0;
            y[64 * c + 32 + l] = d1 * (float)(qs[32 * c + l] >> 4) - mm1;
        }
    }
}

/* block_q6_K: u8 ql[128], u8 qh[64], i8 scales[16], fp16 d.
 * Two halves of 128; in half h, for l in 0..31, the four 6-bit values at
 * y[l], y[l+32], y[l+64], y[l+96] take their low 4 bits from ql (low/high
 * nibble of ql[l] and ql[l+32]) and high 2 bits from qh[l] bit pairs 0,1,2,3;
 * q is offset by -32 and scaled by d*scales[sub-block of 16]. */
static void dq_q6_k_block(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    uint16_t dh;
    memcpy(&dh, b + 208, 2);
    const float d = or_f16_to_f32(dh);
    for (int h = 0; h < 2; ++h) {
        const uint8_t* L = ql + 64 * h;
        const uint8_t* Hh = qh + 32 * h;
        const int8_t* S = sc + 8 * h;
        float* Y = y + 128 * h;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int)((L[l] & 0x0f) | (((Hh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((L[l + 32] & 0x0f) | (((Hh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((L[l] >> 4) | (((Hh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((L[l + 32] >> 4) | (((Hh[l] >> 6) & 3) << 4)) - 32;
            Y[l] = d * (float)S[is + 0] * (float)q1;
            Y[l + 32] = d * (float)S[is + 2] * (float)q2;
            Y[l + 64] = d * (float)S[is + 4] * (float)q3;
            Y[l + 96] = d * (float)S[is + 6] * (float)q4;
        }
    }
}

int or_dequant(int type, const void* src, int64_t n, float* dst) {
    const uint8_t* s = (const uint8_t*)src;
    int64_t be = or_type_block_elems(type);
    if (be <= 0 || n % be) return -1;
    int64_t nb = n / be, bb = or_type_block_bytes(type);
    switch (type) {
        case OR_T_Q8_0:
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < nb; ++i) dq_q8_0_block(s + i * bb, dst + i * 32);
            return 0;
        case OR_T_Q4_K:
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < nb; ++i) dq_q4_k_block(s + i * bb, dst + i * 256);
            return 0;
        case OR_T_Q6_K:
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < nb; ++i) dq_q6_k_block(s + i * bb, dst + i * 256);
            return 0;
        case OR_T_F32:
            memcpy(dst, src, (size_t)n * 4);
            return 0;
        case OR_T_F16: {
            const uint16_t* h = (const uint16_t*)src;
            for (int64_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(h[i]);
            return 0;
        }
        case OR_T_BF16: {
            const uint16_t* h = (const uint16_t*)src;
            for (int64_t i = 0; i < n; ++i) dst[i] = or_bf16_to_f32(h[i]);
            return 0;
        }
        default: return -1;
    }
}

/* ------------------------------------------------------------------------- */
/* GGUF v3 reader                                                             */
/* ------------------------------------------------------------------------- */

enum { GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };

typedef struct {
    char* key;
    int type;
    int arr_type;
    int64_t arr_len;
    int64_t i;
    double f;
    char* s;
} or_kv;

typedef struct {
    char* name;
    int type;
    int ndims;
    int64_t dims[4];
    uint64_t offset;
    int64_t nbytes;
    const uint8_t* data;
} or_tinfo;

struct or_gguf {
    uint8_t* owned;
    const uint8_t* base;
    size_t size;
    int64_t n_kv, n_t;
    or_kv* kv;
    or_tinfo* t;
};

static char g_err[512];
const char* or_gguf_error(void) { return g_err; }

typedef struct { const uint8_t* p; const uint8_t* end; int bad; } rd;
static int rd_need(rd* r, size_t n) {
    if (r->bad || (size_t)(r->end - r->p) < n) { r->bad = 1; return 0; }
    return 1;
}
static uint64_t rd_u(rd* r, int n) {
    if (!rd_need(r, (size_t)n)) return 0;
    uint64_t v = 0;
    memcpy(&v, r->p, (size_t)n); /* little-endian host */
    r->p += n;
    return v;
}
static char* rd_str(rd* r) {
    uint64_t len = rd_u(r, 8);
    if (r->bad || len > (uint64_t)(r->end - r->p)) { r->bad = 1; return NULL; }
    char* s = (char*)malloc(len + 1);
    memcpy(s, r->p, len);
    s[len] = 0;
    r->p += len;
    return s;
}
static int gv_size(int t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        default: return 0;
    }
}
/* Steps over one encoded value of type t (gguf.md: strings are a u64 length
 * and bytes, arrays a u32 element type, a u64 count and the elements). */
static void rd_skip(rd* r, int t, int depth) {
    if (t == GV_STR) {
        uint64_t len = rd_u(r, 8);
        if (rd_need(r, len)) r->p += len;
    } else if (t == GV_ARR) {
        int et = (int)rd_u(r, 4);
        uint64_t n = rd_u(r, 8);
        if (depth > 8 || n > (uint64_t)(r->end - r->p)) { r->bad = 1; return; }
        for (uint64_t k = 0; k < n && !r->bad; ++k) rd_skip(r, et, depth + 1);
    } else if (gv_size(t) > 0) {
        if (rd_need(r, (size_t)gv_size(t))) r->p += gv_size(t);
    } else {
        r->bad = 1;
    }
}
static void rd_scalar(rd* r, int t, int64_t* iv, double* fv) {
    uint64_t raw = rd_u(r, gv_size(t));
    switch (t) {
        case GV_U8: *iv = (uint8_t)raw; break;
        case GV_I8: *iv = (int8_t)raw; break;
        case GV_U16: *iv = (uint16_t)raw; break;
        case GV_I16: *iv = (int16_t)raw; break;
        case GV_U32: *iv = (uint32_t)raw; break;
        case GV_I32: *iv = (int32_t)raw; break;
        case GV_U64: *iv = (int64_t)raw; break;
        case GV_I64: *iv = (int64_t)raw; break;
        case GV_BOOL: *iv = raw ? 1 : 0; break;
        case GV_F32: { uint32_t b = (uint32_t)raw; float f; memcpy(&f, &b, 4); *fv = f; break; }
        case GV_F64: { double d; memcpy(&d, &raw, 8); *fv = d; break; }
        default: break;
    }
    if (t == GV_F32 || t == GV_F64) *iv = (int64_t)*fv; else *fv = (double)*iv;
}

void or_gguf_close(or_gguf* g) {
    if (!g) return;
    for (int64_t i = 0; i < g->n_kv; ++i) { free(g->kv[i].key); free(g->kv[i].s); }
    for (int64_t i = 0; i < g->n_t; ++i) free(g->t[i].name);
    free(g->kv);
    free(g->t);
    free(g->owned);
    free(g);
}

static or_gguf* parse(or_gguf* g) {
    rd r = {g->base, g->base + g->size, 0};
    if (g->size < 24 || memcmp(g->base, "GGUF", 4) != 0) {
        snprintf(g_err, sizeof g_err, "gguf: bad magic");
        or_gguf_close(g);
        return NULL;
    }
    r.p += 4;
    uint32_t ver = (uint32_t)rd_u(&r, 4);
    if (ver != 3) {
        snprintf(g_err, sizeof g_err, "gguf: unsupported version %u", ver);
        or_gguf_close(g);
        return NULL;
    }
    g->n_t = (int64_t)rd_u(&r, 8);
    g->n_kv = (int64_t)rd_u(&r, 8);
    if (g->n_t < 0 || g->n_kv < 0 || g->n_t > (1 << 24) || g->n_kv > (1 << 24)) {
        snprintf(g_err, sizeof g_err, "gguf: bad counts");
        g->n_t = g->n_kv = 0;
        or_gguf_close(g);
        return NULL;
    }
    g->kv = (or_kv*)calloc((size_t)g->n_kv + 1, sizeof(or_kv));
    g->t = (or_tinfo*)calloc((size_t)g->n_t + 1, sizeof(or_tinfo));
    uint64_t alignment = 32;
    for (int64_t i = 0; i < g->n_kv && !r.bad; ++i) {
        or_kv* kv = &g->kv[i];
        kv->key = rd_str(&r);
        kv->type = (int)rd_u(&r, 4);
        if (kv->type == GV_STR) {
            kv->s = rd_str(&r);
        } else if (kv->type == GV_ARR) {
            kv->arr_type = (int)rd_u(&r, 4);
            uint64_t n = rd_u(&r, 8);
            if (n > (uint64_t)(r.end - r.p)) r.bad = 1; /* every element is at least one byte */
            kv->arr_len = (int64_t)n;
            for (uint64_t k = 0; k < n && !r.bad; ++k) rd_skip(&r, kv->arr_type, 1);
        } else if (gv_size(kv->type) > 0) {
            rd_scalar(&r, kv->type, &kv->i, &kv->f);
        } else {
            r.bad = 1;
        }
        if (!r.bad && kv->key && strcmp(kv->key, "general.alignment") == 0) {
            if (kv->type != GV_U32 && kv->type != GV_U64) r.bad = 1;
            alignment = (uint64_t)kv->i;
        }
    }
    for (int64_t i = 0; i < g->n_t && !r.bad; ++i) {
        or_tinfo* t = &g->t[i];
        t->name = rd_str(&r);
        t->ndims = (int)rd_u(&r, 4);
        if (t->ndims < 1 || t->ndims > 4) { r.bad = 1; break; }
        for (int d = 0; d < 4; ++d) t->dims[d] = 1;
        for (int d = 0; d < t->ndims; ++d) {
            uint64_t x = rd_u(&r, 8);
            if (x == 0 || x > ((uint64_t)1 << 40)) r.bad = 1; /* zero or implausible: no product can wrap */
            t->dims[d] = (int64_t)x;
        }
        t->type = (int)rd_u(&r, 4);
        t->offset = rd_u(&r, 8);
    }
    /* the spec asks for a multiple of 8 (docs/gguf.md, general.alignment) */
    if (r.bad || alignment == 0 || alignment % 8 != 0 || alignment > ((uint64_t)1 << 20)) {
        snprintf(g_err, sizeof g_err, "gguf: truncated or malformed header");
        or_gguf_close(g);
        return NULL;
    }
    size_t hdr = (size_t)(r.p - g->base);
    size_t data0 = (hdr + alignment - 1) / alignment * alignment;
    for (int64_t i = 0; i < g->n_t; ++i) {
        or_tinfo* t = &g->t[i];
        int64_t n = 1;
        int wrap = 0;
        for (int d = 0; d < 4; ++d) wrap |= __builtin_mul_overflow(n, t->dims[d], &n);
        int64_t rb = or_row_bytes(t->type, t->dims[0]);
        if (rb < 0) {
            snprintf(g_err, sizeof g_err, "gguf: tensor %s has unsupported type %d or ragged row", t->name, t->type);
            or_gguf_close(g);
            return NULL;
        }
        uint64_t rows = (uint64_t)(n / t->dims[0]);
        uint64_t room = g->size > data0 ? g->size - data0 : 0;
        if (wrap || n <= 0 ||
            (rows != 0 && (uint64_t)rb > UINT64_MAX / rows)) {
            snprintf(g_err, sizeof g_err, "gguf: tensor %s size overflows", t->name);
            or_gguf_close(g);
            return NULL;
        }
        t->nbytes = (int64_t)((uint64_t)rb * rows);
        if (t->offset % alignment != 0 || t->offset > room || (uint64_t)t->nbytes > room - t->offset) {
            snprintf(g_err, sizeof g_err, "gguf: tensor %s data out of range", t->name);
            or_gguf_close(g);
            return NULL;
        }
        t->data = g->base + data0 + t->offset;
    }
    return g;
}

or_gguf* or_gguf_open(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) {
        snprintf(g_err, sizeof g_err, "gguf: cannot open %s", path);
        return NULL;
    }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    or_gguf* g = (or_gguf*)calloc(1, sizeof(or_gguf));
    g->owned = (uint8_t*)malloc((size_t)sz + 1);
    if (fread(g->owned, 1, (size_t)sz, f) != (size_t)sz) {
        fclose(f);
        snprintf(g_err, sizeof g_err, "gguf: short read");
        or_gguf_close(g);
        return NULL;
    }
    fclose(f);
    g->base = g->owned;
    g->size = (size_t)sz;
    return parse(g);
}

or_gguf* or_gguf_open_memory(const void* data, size_t size) {
    or_gguf* g = (or_gguf*)calloc(1, sizeof(or_gguf));
    g->base = (const uint8_t*)data;
    g->size = size;
    return parse(g);
}

int64_t or_gguf_n_tensors(const or_gguf* g) { return g->n_t; }
int64_t or_gguf_find_tensor(const or_gguf* g, const char* name) {
    for (int64_t i = 0; i < g->n_t; ++i)
        if (strcmp(g->t[i].name, name) == 0) return i;
    return -1;
}
const char* or_gguf_tensor_name(const or_gguf* g, int64_t i) { return g->t[i].name; }
int or_gguf_tensor_type(const or_gguf* g, int64_t i) { return g->t[i].type; }
int or_gguf_tensor_ndims(const or_gguf* g, int64_t i) { return g->t[i].ndims; }
int64_t or_gguf_tensor_dim(const or_gguf* g, int64_t i, int d) { return g->t[i].dims[d]; }
const void* or_gguf_tensor_data(const or_gguf* g, int64_t i) { return g->t[i].data; }
int64_t or_gguf_tensor_nbytes(const or_gguf* g, int64_t i) { return g->t[i].nbytes; }

static const or_kv* find_kv(const or_gguf* g, const char* key) {
    for (int64_t i = 0; i < g->n_kv; ++i)
        if (g->kv[i].key && strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
    return NULL;
}
int or_gguf_meta_int(const or_gguf* g, const char* key, int64_t* out) {
    const or_kv* kv = find_kv(g, key);
    if (!kv || kv->type == GV_STR || kv->type == GV_ARR || kv->type == GV_F32 || kv->type == GV_F64) return -1;
    *out = kv->i;
    return 0;
}
int or_gguf_meta_f64(const or_gguf* g, const char* key, double* out) {
    const or_kv* kv = find_kv(g, key);
    if (!kv || (kv->type != GV_F32 && kv->type != GV_F64)) return -1;
    *out = kv->f;
    return 0;
}
int or_gguf_meta_str(const or_gguf* g, const char* key, const char** out) {
    const or_kv* kv = find_kv(g, key);
    if (!kv || kv->type != GV_STR) return -1;
    *out = kv->s;
    return 0;
}
int or_gguf_meta_array_len(const or_gguf* g, const char* key, int64_t* out) {
    const or_kv* kv = find_kv(g, key);
    if (!kv || kv->type != GV_ARR) return -1;
    *out = kv->arr_len;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* FP32 ops                                                                   */
/* ------------------------------------------------------------------------- */

int or_num_threads(void) { return omp_get_max_threads(); }

/* rms_norm_forward: y = x * (mean(x^2) + eps)^-1/2 * gamma, per row
 * (dense_decoder.cpp:559, :622, :652; per-head use :540-550). */
void or_rms_norm(const float* x, const float* gamma, float eps, float* y, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * cols;
        double ss = 0.0;
        for (int c = 0; c < cols; ++c) ss += (double)xr[c] * xr[c];
        const float inv = (float)(1.0 / sqrt(ss / cols + (double)eps));
        for (int c = 0; c < cols; ++c) y[(size_t)r * cols + c] = xr[c] * inv * gamma[c];
    }
}

/* rope_forward (dense_decoder.cpp:587-590): in each head, pairs (2i, 2i+1)
 * rotate by angle (pos0+r) * theta^(-2i/hd) (exponent as brolm's host
 * inv_freq, src/qwen3vl_text.cpp:265-277). Angles and sin/cos in double. */
void or_rope(float* x, int rows, int hd, int n_heads, int pos0, float theta) {
    const int half = hd / 2;
    for (int r = 0; r < rows; ++r) {
        const double pos = (double)(pos0 + r);
        for (int i = 0; i < half; ++i) {
            const double inv = pow((double)theta, -2.0 * i / (double)hd);
            const double a = pos * inv;
            const double c = cos(a), s = sin(a);
            for (int h = 0; h < n_heads; ++h) {
                float* p = x + (size_t)r * n_heads * hd + (size_t)h * hd + 2 * i;
                const double x0 = p[0], x1 = p[1];
                p[0] = (float)(x0 * c - x1 * s);
                p[1] = (float)(x0 * s + x1 * c);
            }
        }
    }
}

static float dot_f32(const float* a, const float* b, int K) {
    float acc[16] = {0};
    int k = 0;
    for (; k + 16 <= K; k += 16)
        for (int j = 0; j < 16; ++j) acc[j] += a[k + j] * b[k + j];
    float s = 0.f;
    for (; k < K; ++k) s += a[k] * b[k];
    for (int j = 0; j < 16; ++j) s += acc[j];
    return s;
}

/* linear_batched without bias (compute.h:54-86): Y = X W^T */
void or_linear(const float* W, const float* X, float* Y, int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const float* w = W + (size_t)n * K;
        for (int m = 0; m < M; ++m) Y[(size_t)m * N + n] = dot_f32(X + (size_t)m * K, w, K);
    }
}

/* flash_attention_decode semantics (dense_decoder.cpp:601-607): scale
 * 1/sqrt(hd) inside, causal (row r sees keys 0..pos0+r), query head h reads
 * KV head h / (n_q/n_kv) (:593-594). Softmax in double. */
void or_attention(const float* q, const float* Kc, const float* Vc, int L, int pos0,
                  int n_q, int n_kv, int hd, float* out) {
    const int group = n_q / n_kv;
    const int kvd = n_kv * hd;
    const double scale = 1.0 / sqrt((double)hd);
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < L; ++r) {
        for (int h = 0; h < n_q; ++h) {
            const int g = h / group;
            const int nk = pos0 + r + 1;
            const float* qv = q + (size_t)r * n_q * hd + (size_t)h * hd;
            double* sc = (double*)malloc(sizeof(double) * (size_t)nk);
            double mx = -1e300;
            for (int j = 0; j < nk; ++j) {
                const float* kv = Kc + (size_t)j * kvd + (size_t)g * hd;
                double s = 0.0;
                for (int d = 0; d < hd; ++d) s += (double)qv[d] * kv[d];
                sc[j] = s * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0.0;
            for (int j = 0; j < nk; ++j) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
            float* o = out + (size_t)r * n_q * hd + (size_t)h * hd;
            for (int d = 0; d < hd; ++d) {
                double a = 0.0;
                for (int j = 0; j < nk; ++j) a += sc[j] * Vc[(size_t)j * kvd + (size_t)g * hd + d];
                o[d] = (float)(a / sum);
            }
            free(sc);
        }
    }
}

float or_silu(float x) { return (float)((double)x / (1.0 + exp(-(double)x))); }

/* ------------------------------------------------------------------------- */
/* Dense decoder (Qwen3 / Mistral 3.1 text)                                   */
/* ------------------------------------------------------------------------- */

typedef struct {
    float *in_ln, *Wq, *Wk, *Wv, *Wo, *q_norm, *k_norm, *post_ln, *Wg, *Wu, *Wd;
    float *Kc, *Vc;
} or_layer;

struct or_model {
    or_config c;
    float* embed;   /* (V, H) */
    float* final_norm;
    float* lm_head; /* (V, H); separate storage even when tied (dense_decoder.cpp:190) */
    or_layer* layers;
    int cache_len, max_seq;
};

static const or_kv* kvx(const or_gguf* g, const char* k) { return find_kv(g, k); }

/* Qwen3Config::from_gguf (src/qwen.cpp:88-149) for "qwen3";
 * Mistral3Config::from_gguf (src/mistral3_config.cpp:130-191) for any other
 * architecture name, whose keys carry that name as prefix ("llama.",
 * "mistral."), with QK-norm off (src/mistral3_text.cpp:26-42) and tying
 * inferred from the absence of output.weight. */
static int load_config(const or_gguf* g, or_config* c) {
    const char* arch = NULL;
    char a[64] = "qwen3";
    if (or_gguf_meta_str(g, "general.architecture", &arch) == 0) snprintf(a, sizeof a, "%s", arch);
    const int qwen = strcmp(a, "qwen3") == 0;
    if (!qwen && strcmp(a, "llama") != 0 && strcmp(a, "mistral") != 0) {
        snprintf(g_err, sizeof g_err, "general.architecture is '%s', expected qwen3, llama or mistral", a);
        return -1;
    }
    int64_t v;
    c->vocab_size = 151936; c->hidden_size = 1024; c->intermediate_size = 3072;
    c->num_hidden_layers = 28; c->num_attention_heads = 16; c->num_key_value_heads = 8;
    c->head_dim = 128; c->rms_norm_eps = 1e-6f; c->rope_theta = 1000000.0f;
    c->tie_word_embeddings = 1; c->max_position_embeddings = 40960;
    if (!qwen) {  /* Mistral3Config::Text defaults (mistral3_config.h:38-58) */
        c->vocab_size = 131072; c->rms_norm_eps = 1e-5f; c->rope_theta = 1.0e9f;
        c->tie_word_embeddings = 0; c->max_position_embeddings = 131072;
    }
    c->use_qk_norm = qwen;
    char key[128];
#define KEY(suffix) (snprintf(key, sizeof key, "%s.%s", a, suffix), key)
#define NEED(suffix, field) \
    if (or_gguf_meta_int(g, KEY(suffix), &v) != 0) { snprintf(g_err, sizeof g_err, "missing metadata '%s'", key); return -1; } \
    c->field = (int)v;
    NEED("embedding_length", hidden_size);
    NEED("feed_forward_length", intermediate_size);
    NEED("block_count", num_hidden_layers);
    NEED("attention.head_count", num_attention_heads);
#undef NEED
    c->num_key_value_heads = or_gguf_meta_int(g, KEY("attention.head_count_kv"), &v) == 0 ? (int)v : c->num_attention_heads;
    c->head_dim = or_gguf_meta_int(g, KEY("attention.key_length"), &v) == 0 ? (int)v
                                                                          : c->hidden_size / c->num_attention_heads;
    double f;
    if (or_gguf_meta_f64(g, KEY("attention.layer_norm_rms_epsilon"), &f) == 0) c->rms_norm_eps = (float)f;
    if (or_gguf_meta_f64(g, KEY("rope.freq_base"), &f) == 0) c->rope_theta = (float)f;
    if (or_gguf_meta_int(g, KEY("context_length"), &v) == 0) c->max_position_embeddings = (int)v;
    if (or_gguf_meta_array_len(g, "tokenizer.ggml.tokens", &v) == 0) c->vocab_size = (int)v;
    else if (or_gguf_meta_int(g, KEY("vocab_size"), &v) == 0) c->vocab_size = (int)v;
    const or_kv* tie = qwen ? kvx(g, "qwen3.tie_word_embeddings") : NULL;
    if (tie && tie->type == GV_BOOL) c->tie_word_embeddings = (int)tie->i;
    else c->tie_word_embeddings = or_gguf_find_tensor(g, "output.weight") < 0;
#undef KEY
    return 0;
}

static float* load_tensor(const or_gguf* g, const char* name, int64_t rows, int64_t cols) {
    int64_t i = or_gguf_find_tensor(g, name);
    if (i < 0) {
        snprintf(g_err, sizeof g_err, "missing tensor '%s'", name);
        return NULL;
    }
    int64_t n = 1;
    for (int d = 0; d < or_gguf_tensor_ndims(g, i); ++d) n *= or_gguf_tensor_dim(g, i, d);
    if (n != rows * cols) {
        snprintf(g_err, sizeof g_err, "tensor '%s': shape mismatch", name);
        return NULL;
    }
    float* out = (float*)malloc(sizeof(float) * (size_t)n);
    if (or_dequant(or_gguf_tensor_type(g, i), or_gguf_tensor_data(g, i), n, out) != 0) {
        free(out);
        snprintf(g_err, sizeof g_err, "tensor '%s': unsupported type", name);
        return NULL;
    }
    return out;
}

/* upload_compute_rope_permuted (weights.h:343-395, permute :104-148): within
 * each head, dst rows (2i, 2i+1) <- src rows (i, i + hd/2). */
static void permute_rows(float* w, int n_heads, int hd, int64_t cols) {
    const int half = hd / 2;
    size_t hb = (size_t)hd * (size_t)cols;
    float* tmp = (float*)malloc(sizeof(float) * hb);
    for (int h = 0; h < n_heads; ++h) {
        float* base = w + (size_t)h * hb;
        for (int i = 0; i < half; ++i) {
            memcpy(tmp + (size_t)(2 * i) * cols, base + (size_t)i * cols, sizeof(float) * (size_t)cols);
            memcpy(tmp + (size_t)(2 * i + 1) * cols, base + (size_t)(i + half) * cols, sizeof(float) * (size_t)cols);
        }
        memcpy(base, tmp, sizeof(float) * hb);
    }
    free(tmp);
}

void or_model_free(or_model* m) {
    if (!m) return;
    for (int l = 0; m->layers && l < m->c.num_hidden_layers; ++l) {
        or_layer* L = &m->layers[l];
        free(L->in_ln); free(L->Wq); free(L->Wk); free(L->Wv); free(L->Wo);
        free(L->q_norm); free(L->k_norm); free(L->post_ln); free(L->Wg); free(L->Wu); free(L->Wd);
        free(L->Kc); free(L->Vc);
    }
    free(m->layers);
    free(m->embed);
    free(m->final_norm);
    free(m->lm_head);
    free(m);
}

/* DenseDecoder ctor checks (dense_decoder.cpp:97-113) + load_weights (:121-192). */
or_model* or_model_load(const or_gguf* g) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    if (load_config(g, &m->c) != 0) { free(m); return NULL; }
    const or_config* c = &m->c;
    if (c->hidden_size <= 0 || c->intermediate_size <= 0 || c->num_hidden_layers <= 0 || c->vocab_size <= 0 ||
        c->head_dim <= 0 || c->num_attention_heads <= 0 || c->num_key_value_heads <= 0 ||
        c->num_attention_heads % c->num_key_value_heads != 0 || c->head_dim % 2 != 0) {
        snprintf(g_err, sizeof g_err, "bad config");
        free(m);
        return NULL;
    }
    const int V = c->vocab_size, H = c->hidden_size, F = c->intermediate_size, HD = c->head_dim;
    const int qd = c->num_attention_heads * HD, kvd = c->num_key_value_heads * HD;
    m->layers = (or_layer*)calloc((size_t)c->num_hidden_layers, sizeof(or_layer));
    char name[128];
#define LOAD(dst, nm, r, cc) do { dst = load_tensor(g, nm, r, cc); if (!dst) { or_model_free(m); return NULL; } } while (0)
    LOAD(m->embed, "token_embd.weight", V, H);
    for (int l = 0; l < c->num_hidden_layers; ++l) {
        or_layer* L = &m->layers[l];
        snprintf(name, sizeof name, "blk.%d.attn_norm.weight", l); LOAD(L->in_ln, name, H, 1);
        snprintf(name, sizeof name, "blk.%d.attn_q.weight", l); LOAD(L->Wq, name, qd, H);
        snprintf(name, sizeof name, "blk.%d.attn_k.weight", l); LOAD(L->Wk, name, kvd, H);
        snprintf(name, sizeof name, "blk.%d.attn_v.weight", l); LOAD(L->Wv, name, kvd, H);
        snprintf(name, sizeof name, "blk.%d.attn_output.weight", l); LOAD(L->Wo, name, H, qd);
        if (c->use_qk_norm) {
            snprintf(name, sizeof name, "blk.%d.attn_q_norm.weight", l); LOAD(L->q_norm, name, HD, 1);
            snprintf(name, sizeof name, "blk.%d.attn_k_norm.weight", l); LOAD(L->k_norm, name, HD, 1);
        }
        snprintf(name, sizeof name, "blk.%d.ffn_norm.weight", l); LOAD(L->post_ln, name, H, 1);
        snprintf(name, sizeof name, "blk.%d.ffn_gate.weight", l); LOAD(L->Wg, name, F, H);
        snprintf(name, sizeof name, "blk.%d.ffn_up.weight", l); LOAD(L->Wu, name, F, H);
        snprintf(name, sizeof name, "blk.%d.ffn_down.weight", l); LOAD(L->Wd, name, H, F);
        permute_rows(L->Wq, c->num_attention_heads, HD, H);
        permute_rows(L->Wk, c->num_key_value_heads, HD, H);
        if (c->use_qk_norm) {
            permute_rows(L->q_norm, 1, HD, 1);
            permute_rows(L->k_norm, 1, HD, 1);
        }
    }
    LOAD(m->final_norm, "output_norm.weight", H, 1);
    if (or_gguf_find_tensor(g, "output.weight") >= 0) {
        LOAD(m->lm_head, "output.weight", V, H);
    } else {
        if (!c->tie_word_embeddings) {
            snprintf(g_err, sizeof g_err, "lm_head.weight missing and tie_word_embeddings is false");
            or_model_free(m);
            return NULL;
        }
        m->lm_head = (float*)malloc(sizeof(float) * (size_t)V * H);
        memcpy(m->lm_head, m->embed, sizeof(float) * (size_t)V * H);
    }
#undef LOAD
    return m;
}

void or_model_config(const or_model* m, or_config* out) { *out = m->c; }

int or_model_allocate_cache(or_model* m, int max_seq_len) {
    if (max_seq_len <= 0) return -1;
    const size_t kvd = (size_t)m->c.num_key_value_heads * m->c.head_dim;
    for (int l = 0; l < m->c.num_hidden_layers; ++l) {
        or_layer* L = &m->layers[l];
        free(L->Kc);
        free(L->Vc);
        L->Kc = (float*)calloc((size_t)max_seq_len * kvd, sizeof(float));
        L->Vc = (float*)calloc((size_t)max_seq_len * kvd, sizeof(float));
    }
    m->max_seq = max_seq_len;
    m->cache_len = 0;
    return 0;
}
void or_model_reset_cache(or_model* m) { m->cache_len = 0; }
/* Benchmark helper: K / V rows [0, len) of every layer get deterministic
 * values in [-1, 1) (an xorshift stream from seed) and cache_len = len, so a
 * decode timing runs at the context of a long prompt without its prefill. */
int or_model_fill_cache(or_model* m, int len, uint64_t seed) {
    if (len < 0 || len > m->max_seq) return -1;
    const size_t kvd = (size_t)m->c.num_key_value_heads * m->c.head_dim;
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (int l = 0; l < m->c.num_hidden_layers; ++l) {
        or_layer* L = &m->layers[l];
        for (size_t i = 0; i < (size_t)len * kvd; ++i) {
            x ^= x << 13; x ^= x >> 7; x ^= x << 17;
            L->Kc[i] = (float)((int64_t)(x >> 40) - (1 << 23)) / (float)(1 << 23);
            x ^= x << 13; x ^= x >> 7; x ^= x << 17;
            L->Vc[i] = (float)((int64_t)(x >> 40) - (1 << 23)) / (float)(1 << 23);
        }
    }
    m->cache_len = len;
    return 0;
}
int or_model_truncate_cache(or_model* m, int len) {
    if (len < 0 || len > m->cache_len) return -1;
    m->cache_len = len;
    return 0;
}
int or_model_cache_len(const or_model* m) { return m->cache_len; }

/* run_layers_ (dense_decoder.cpp:526-681) in FP32. */
int or_model_forward(or_model* m, const int32_t* ids, int L, int last_only, float* logits, float* hidden) {
    const or_config* c = &m->c;
    if (!ids || L <= 0) { snprintf(g_err, sizeof g_err, "forward: bad ids / L"); return -1; }
    if (m->max_seq == 0) { snprintf(g_err, sizeof g_err, "forward: cache not allocated"); return -1; }
    if (m->cache_len + L > m->max_seq) { snprintf(g_err, sizeof g_err, "forward: capacity"); return -1; }
    for (int i = 0; i < L; ++i)
        if (ids[i] < 0 || ids[i] >= c->vocab_size) { snprintf(g_err, sizeof g_err, "forward: id out of range"); return -1; }
    const int H = c->hidden_size, F = c->intermediate_size, HD = c->head_dim;
    const int nq = c->num_attention_heads, nkv = c->num_key_value_heads;
    const int qd = nq * HD, kvd = nkv * HD, V = c->vocab_size;
    const int pos0 = m->cache_len;
    const float eps = c->rms_norm_eps;
    float* h = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* nrm = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* q = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* k = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* v = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* qn = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* kn = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* att = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* proj = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* gt = (float*)malloc(sizeof(float) * (size_t)L * F);
    float* up = (float*)malloc(sizeof(float) * (size_t)L * F);
    for (int i = 0; i < L; ++i) memcpy(h + (size_t)i * H, m->embed + (size_t)ids[i] * H, sizeof(float) * H);
    for (int l = 0; l < c->num_hidden_layers; ++l) {
        or_layer* Ly = &m->layers[l];
        or_rms_norm(h, Ly->in_ln, eps, nrm, L, H);
        or_linear(Ly->Wq, nrm, q, L, qd, H);
        or_linear(Ly->Wk, nrm, k, L, kvd, H);
        or_linear(Ly->Wv, nrm, v, L, kvd, H);
        if (c->use_qk_norm) {
            or_rms_norm(q, Ly->q_norm, eps, qn, L * nq, HD);
            or_rms_norm(k, Ly->k_norm, eps, kn, L * nkv, HD);
        } else {
            memcpy(qn, q, sizeof(float) * (size_t)L * qd);
            memcpy(kn, k, sizeof(float) * (size_t)L * kvd);
        }
        or_rope(qn, L, HD, nq, pos0, c->rope_theta);
        or_rope(kn, L, HD, nkv, pos0, c->rope_theta);
        memcpy(Ly->Kc + (size_t)pos0 * kvd, kn, sizeof(float) * (size_t)L * kvd);
        memcpy(Ly->Vc + (size_t)pos0 * kvd, v, sizeof(float) * (size_t)L * kvd);
        or_attention(qn, Ly->Kc, Ly->Vc, L, pos0, nq, nkv, HD, att);
        or_linear(Ly->Wo, att, proj, L, H, qd);
        for (size_t i = 0; i < (size_t)L * H; ++i) h[i] += proj[i];
        or_rms_norm(h, Ly->post_ln, eps, nrm, L, H);
        or_linear(Ly->Wg, nrm, gt, L, F, H);
        or_linear(Ly->Wu, nrm, up, L, F, H);
        for (size_t i = 0; i < (size_t)L * F; ++i) gt[i] = or_silu(gt[i]) * up[i];
        or_linear(Ly->Wd, gt, proj, L, H, F);
        for (size_t i = 0; i < (size_t)L * H; ++i) h[i] += proj[i];
    }
    or_rms_norm(h, m->final_norm, eps, nrm, L, H);
    if (hidden) memcpy(hidden, nrm, sizeof(float) * (size_t)L * H);
    if (logits) {
        if (last_only) or_linear(m->lm_head, nrm + (size_t)(L - 1) * H, logits, 1, V, H);
        else or_linear(m->lm_head, nrm, logits, L, V, H);
    }
    m->cache_len += L;
    free(h); free(nrm); free(q); free(k); free(v); free(qn); free(kn); free(att); free(proj); free(gt); free(up);
    return 0;
}

/* DenseDecoder::forward_encode / run_layers_encode_ (dense_decoder.cpp:296-309,
 * :682-779) in FP32: the same layers with RoPE positions 0..L-1, every row
 * attending all L keys (no causal limit, no KV cache), no lm_head.  hidden:
 * (L, H) post-final-norm.  The cache is not touched. */
int or_model_forward_encode(or_model* m, const int32_t* ids, int L, float* hidden) {
    const or_config* c = &m->c;
    if (!ids || L <= 0 || !hidden) { snprintf(g_err, sizeof g_err, "forward_encode: bad arguments"); return -1; }
    for (int i = 0; i < L; ++i)
        if (ids[i] < 0 || ids[i] >= c->vocab_size) { snprintf(g_err, sizeof g_err, "forward_encode: id out of range"); return -1; }
    const int H = c->hidden_size, F = c->intermediate_size, HD = c->head_dim;
    const int nq = c->num_attention_heads, nkv = c->num_key_value_heads;
    const int qd = nq * HD, kvd = nkv * HD;
    const float eps = c->rms_norm_eps;
    float* h = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* nrm = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* q = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* k = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* v = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* qn = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* kn = (float*)malloc(sizeof(float) * (size_t)L * kvd);
    float* att = (float*)malloc(sizeof(float) * (size_t)L * qd);
    float* proj = (float*)malloc(sizeof(float) * (size_t)L * H);
    float* gt = (float*)malloc(sizeof(float) * (size_t)L * F);
    float* up = (float*)malloc(sizeof(float) * (size_t)L * F);
    for (int i = 0; i < L; ++i) memcpy(h + (size_t)i * H, m->embed + (size_t)ids[i] * H, sizeof(float) * H);
    for (int l = 0; l < c->num_hidden_layers; ++l) {
        or_layer* Ly = &m->layers[l];
        or_rms_norm(h, Ly->in_ln, eps, nrm, L, H);
        or_linear(Ly->Wq, nrm, q, L, qd, H);
        or_linear(Ly->Wk, nrm, k, L, kvd, H);
        or_linear(Ly->Wv, nrm, v, L, kvd, H);
        if (c->use_qk_norm) {
            or_rms_norm(q, Ly->q_norm, eps, qn, L * nq, HD);
            or_rms_norm(k, Ly->k_norm, eps, kn, L * nkv, HD);
        } else {
            memcpy(qn, q, sizeof(float) * (size_t)L * qd);
            memcpy(kn, k, sizeof(float) * (size_t)L * kvd);
        }
        or_rope(qn, L, HD, nq, 0, c->rope_theta);
        or_rope(kn, L, HD, nkv, 0, c->rope_theta);
        /* one row at a time as the last of L positions: keys 0..L-1 */
        for (int i = 0; i < L; ++i)
            or_attention(qn + (size_t)i * qd, kn, v, 1, L - 1, nq, nkv, HD, att + (size_t)i * qd);
        or_linear(Ly->Wo, att, proj, L, H, qd);
        for (size_t i = 0; i < (size_t)L * H; ++i) h[i] += proj[i];
        or_rms_norm(h, Ly->post_ln, eps, nrm, L, H);
        or_linear(Ly->Wg, nrm, gt, L, F, H);
        or_linear(Ly->Wu, nrm, up, L, F, H);
        for (size_t i = 0; i < (size_t)L * F; ++i) gt[i] = or_silu(gt[i]) * up[i];
        or_linear(Ly->Wd, gt, proj, L, H, F);
        for (size_t i = 0; i < (size_t)L * H; ++i) h[i] += proj[i];
    }
    or_rms_norm(h, m->final_norm, eps, hidden, L, H);
    free(h); free(nrm); free(q); free(k); free(v); free(qn); free(kn); free(att); free(proj); free(gt); free(up);
    return 0;
}

const float* or_model_weight(const or_model* m, int layer, const char* which, int64_t* rows, int64_t* cols) {
    const or_config* c = &m->c;
    const int H = c->hidden_size, F = c->intermediate_size, HD = c->head_dim;
    const int qd = c->num_attention_heads * HD, kvd = c->num_key_value_heads * HD;
    if (strcmp(which, "embed") == 0) { *rows = c->vocab_size; *cols = H; return m->embed; }
    if (strcmp(which, "lm_head") == 0) { *rows = c->vocab_size; *cols = H; return m->lm_head; }
    if (strcmp(which, "final_norm") == 0) { *rows = H; *cols = 1; return m->final_norm; }
    if (layer < 0 || layer >= c->num_hidden_layers) return NULL;
    const or_layer* L = &m->layers[layer];
    if (strcmp(which, "in_ln") == 0) { *rows = H; *cols = 1; return L->in_ln; }
    if (strcmp(which, "post_ln") == 0) { *rows = H; *cols = 1; return L->post_ln; }
    if (strcmp(which, "q") == 0) { *rows = qd; *cols = H; return L->Wq; }
    if (strcmp(which, "k") == 0) { *rows = kvd; *cols = H; return L->Wk; }
    if (strcmp(which, "v") == 0) { *rows = kvd; *cols = H; return L->Wv; }
    if (strcmp(which, "o") == 0) { *rows = H; *cols = qd; return L->Wo; }
    if (strcmp(which, "q_norm") == 0) { *rows = HD; *cols = 1; return L->q_norm; }
    if (strcmp(which, "k_norm") == 0) { *rows = HD; *cols = 1; return L->k_norm; }
    if (strcmp(which, "gate") == 0) { *rows = F; *cols = H; return L->Wg; }
    if (strcmp(which, "up") == 0) { *rows = F; *cols = H; return L->Wu; }
    if (strcmp(which, "down") == 0) { *rows = H; *cols = F; return L->Wd; }
    return NULL;
}

/* argmax (src/detail/generate.cpp:38-48): strict '>' keeps the lowest index. */
int or_argmax(const float* logits, int vocab, float* margin) {
    int best = 0;
    float bv = logits[0], second = -INFINITY;
    for (int i = 1; i < vocab; ++i) {
        if (logits[i] > bv) { second = bv; bv = logits[i]; best = i; }
        else if (logits[i] > second) second = logits[i];
    }
    if (margin) *margin = bv - second;
    return best;
}

/* sample_token (src/detail/generate.cpp:68-142) with the uniform draw u in
 * [0, 1) supplied by the caller (the reference draws it from
 * uniform_real_distribution<double>(0, 1) over its std::mt19937_64):
 *   greedy (T <= 0 or top_k == 1): the strict-'>' argmax;
 *   p_i = float(exp(float(l_i * (1/T)) - max)) * float(1 / sum), sum in double;
 *   order = indices by descending p; equal p keep ascending index (the
 *     reference's std::sort leaves that order unspecified);
 *   keep = top_k, then the shortest prefix whose running double sum reaches
 *     top_p (at least 1); r = u * (double sum of the kept p);
 *   the first kept index whose running sum exceeds r, else the last kept.
 * margin (optional): distance of r to the nearer end of the chosen token's
 * interval, as a fraction of the kept mass (0 for greedy). */
static const float* g_sort_p;
static int cmp_desc_p(const void* a, const void* b) {
    const int i = *(const int*)a, j = *(const int*)b;
    const float pi = g_sort_p[i], pj = g_sort_p[j];
    if (pi > pj) return -1;
    if (pi < pj) return 1;
    return (i > j) - (i < j);
}
int or_sample_token(const float* logits, int vocab, float temperature, int top_k, float top_p, double u,
                    double* margin) {
    if (margin) *margin = 0.0;
    if (vocab <= 0) return 0;
    if (temperature <= 0.0f || top_k == 1) return or_argmax(logits, vocab, NULL);
    const float inv_t = 1.0f / temperature;
    float mx = logits[0] * inv_t;
    for (int i = 1; i < vocab; ++i) {
        const float x = logits[i] * inv_t;
        if (x > mx) mx = x;
    }
    float* p = (float*)malloc(sizeof(float) * (size_t)vocab);
    int* order = (int*)malloc(sizeof(int) * (size_t)vocab);
    double sum = 0.0;
    for (int i = 0; i < vocab; ++i) {
        p[i] = expf(logits[i] * inv_t - mx);
        sum += p[i];
    }
    const float norm = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
    for (int i = 0; i < vocab; ++i) {
        p[i] *= norm;
        order[i] = i;
    }
    g_sort_p = p;
    qsort(order, (size_t)vocab, sizeof(int), cmp_desc_p);
    int keep = vocab;
    if (top_k > 0 && top_k < keep) keep = top_k;
    if (top_p < 1.0f) {
        double cum = 0.0;
        int nucleus = 0;
        for (int i = 0; i < keep; ++i) {
            cum += p[order[i]];
            ++nucleus;
            if (cum >= (double)top_p) break;
        }
        keep = nucleus > 1 ? nucleus : 1;
    }
    double kept = 0.0;
    for (int i = 0; i < keep; ++i) kept += p[order[i]];
    int tok = order[0];
    if (kept > 0.0) {
        const double r = u * kept;
        double acc = 0.0, lo = 0.0;
        tok = order[keep - 1];
        int found = 0;
        for (int i = 0; i < keep; ++i) {
            lo = acc;
            acc += p[order[i]];
            if (r < acc) {
                tok = order[i];
                found = 1;
                break;
            }
        }
        if (margin) {
            const double a = found ? r - lo : r - (acc - p[order[keep - 1]]);
            const double b = found ? acc - r : 0.0;
            *margin = (a < b ? a : b) / kept;
        }
    }
    free(p);
    free(order);
    return tok;
}

/* generate (include/brolm/detail/generate.h:78-123), greedy sampling. */
int or_generate_greedy(or_model* m, const int32_t* prompt, int n_prompt, int max_new, int eos_id, int32_t* out,
                       float* margins) {
    if (n_prompt <= 0 || max_new <= 0) return 0;
    const int V = m->c.vocab_size;
    if (or_model_allocate_cache(m, n_prompt + max_new) != 0) return -1;
    float* lg = (float*)malloc(sizeof(float) * (size_t)V);
    if (or_model_forward(m, prompt, n_prompt, 1, lg, NULL) != 0) { free(lg); return -1; }
    int n = 0;
    float mg;
    int next = or_argmax(lg, V, &mg);
    const int stop = eos_id >= 0;
    if (!(stop && next == eos_id)) {
        if (margins) margins[n] = mg;
        out[n++] = next;
        while (n < max_new) {
            int32_t cur = out[n - 1];
            if (or_model_forward(m, &cur, 1, 1, lg, NULL) != 0) { free(lg); return -1; }
            next = or_argmax(lg, V, &mg);
            if (stop && next == eos_id) break;
            if (margins) margins[n] = mg;
            out[n++] = next;
        }
    }
    free(lg);
    return n;
}
