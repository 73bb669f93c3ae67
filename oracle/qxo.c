/* ORACLE — test infrastructure only (see qxo.h).  Scalar restatement of the
 * reference's f32 path; line numbers are of the reference's src/qx_format.c. */
#define _GNU_SOURCE
#include "qxo.h"
#include "qx_grids.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* built with -ffp-contract=off: no a*b+c fusion anywhere in this file */

uint64_t qxo_fnv1a64(const void *p, uint64_t n) {
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = 1469598103934665603ull;
    for (uint64_t i = 0; i < n; ++i) { h ^= b[i]; h *= 1099511628211ull; }
    return h;
}

/* :1854-1876 — exact widening; exponent 31 (inf/NaN) maps to +-65504 */
float qxo_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x477fe000u;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

static uint8_t ksign(uint32_t i) { return (uint8_t)(i | ((uint32_t)(__builtin_popcount(i) & 1) << 7)); }
static uint8_t iq2_grid_byte(uint32_t idx, int j) { return qx_iq2xs_levels[(qx_iq2xs_packed[idx] >> (2 * j)) & 3]; }
static uint8_t iq3_grid_byte(uint32_t idx, int j) { return qx_iq3xxs_levels[(qx_iq3xxs_packed[idx] >> (3 * j)) & 7]; }
static uint8_t iq2s_grid_byte(uint32_t idx, int j) { return qx_iq2xs_levels[(qx_iq2s_packed[idx] >> (2 * j)) & 3]; }
static uint8_t iq3s_grid_byte(uint32_t idx, int j) { return qx_iq3s_levels[(qx_iq3s_packed[idx] >> (3 * j)) & 7]; }

/* :1914-1933 */
static void dec_iq2_xs(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b));
    for (int ib = 0; ib < 8; ++ib) {
        const uint8_t s = b[66 + ib];
        const float db0 = (d * (0.5f + (float)(s & 15))) * 0.25f;
        const float db1 = (d * (0.5f + (float)(s >> 4))) * 0.25f;
        for (int l = 0; l < 4; ++l) {
            const uint16_t q = rd16(b + 2 + 2 * (4 * ib + l));
            const uint8_t sg = ksign(q >> 9);
            const float db = l < 2 ? db0 : db1;
            for (int j = 0; j < 8; ++j)
                y[32 * ib + 8 * l + j] = (db * (float)iq2_grid_byte(q & 511u, j)) * ((sg >> j) & 1 ? -1.0f : 1.0f);
        }
    }
}

/* :1935-1959 */
static void dec_iq3_xxs(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b));
    const uint8_t *qs = b + 2;
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t a = rd32(b + 66 + 4 * ib);
        const float db = (d * (0.5f + (float)(a >> 28))) * 0.5f;
        for (int l = 0; l < 4; ++l) {
            const uint8_t sg = ksign((a >> (7 * l)) & 127u);
            const uint8_t i1 = qs[8 * ib + 2 * l], i2 = qs[8 * ib + 2 * l + 1];
            for (int j = 0; j < 4; ++j) {
                y[32 * ib + 8 * l + j] = (db * (float)iq3_grid_byte(i1, j)) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                y[32 * ib + 8 * l + j + 4] = (db * (float)iq3_grid_byte(i2, j)) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
            }
        }
    }
}

/* :1961-1984 — 10-bit grid index (qs byte + 2 bits of qh), explicit sign bytes */
static void dec_iq2_s(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *sg = b + 34, *qh = b + 66, *sc = b + 74;
    for (int ib = 0; ib < 8; ++ib) {
        const float db0 = (d * (0.5f + (float)(sc[ib] & 15))) * 0.25f;
        const float db1 = (d * (0.5f + (float)(sc[ib] >> 4))) * 0.25f;
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = (uint32_t)qs[4 * ib + l] | (((uint32_t)qh[ib] << (8 - 2 * l)) & 0x300u);
            const float db = l < 2 ? db0 : db1;
            for (int j = 0; j < 8; ++j)
                y[32 * ib + 8 * l + j] = (db * (float)iq2s_grid_byte(idx, j)) * ((sg[4 * ib + l] >> j) & 1 ? -1.0f : 1.0f);
        }
    }
}

/* :1986-2030 — 9-bit grid index (qs byte + 1 bit of qh), explicit sign bytes,
 * scale d*(1+2s) per 32 values */
static void dec_iq3_s(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *qh = b + 66, *sg = b + 74, *sc = b + 106;
    for (int ib = 0; ib < 8; ++ib) {
        const float db = d * (1.0f + 2.0f * (float)((sc[ib / 2] >> (4 * (ib & 1))) & 15));
        for (int l = 0; l < 4; ++l) {
            const uint32_t i1 = (uint32_t)qs[8 * ib + 2 * l] | (((uint32_t)qh[ib] << (8 - 2 * l)) & 256u);
            const uint32_t i2 = (uint32_t)qs[8 * ib + 2 * l + 1] | (((uint32_t)qh[ib] << (7 - 2 * l)) & 256u);
            const uint8_t s8 = sg[4 * ib + l];
            for (int j = 0; j < 4; ++j) {
                y[32 * ib + 8 * l + j] = (db * (float)iq3s_grid_byte(i1, j)) * ((s8 >> j) & 1 ? -1.0f : 1.0f);
                y[32 * ib + 8 * l + j + 4] = (db * (float)iq3s_grid_byte(i2, j)) * ((s8 >> (j + 4)) & 1 ? -1.0f : 1.0f);
            }
        }
    }
}

/* :2032-2053 */
static void dec_iq4_xs(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b));
    const uint16_t sh = rd16(b + 2);
    const uint8_t *sl = b + 4, *qs = b + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; ++j) {
            y[32 * ib + j] = dl * (float)qx_iq4nl_values[qs[16 * ib + j] & 15];
            y[32 * ib + 16 + j] = dl * (float)qx_iq4nl_values[qs[16 * ib + j] >> 4];
        }
    }
}

/* :2079-2110 */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else { *d = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4)); *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4)); }
}

/* :2112-2145 — 5-bit codes: nibble of qs plus bit (2j or 2j+1) of qh[l] */
static void dec_q5_k(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b)), dmin = qxo_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *qh = b + 16, *q = b + 48;
    for (int j = 0; j < 4; ++j) {
        uint8_t s, m;
        scale_min_k4(2 * j, sc, &s, &m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        scale_min_k4(2 * j + 1, sc, &s, &m);
        const float d2 = d * (float)s, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l)
            y[64 * j + l] = d1 * (float)((q[32 * j + l] & 15) | (((qh[l] >> (2 * j)) & 1) << 4)) - m1;
        for (int l = 0; l < 32; ++l)
            y[64 * j + 32 + l] = d2 * (float)((q[32 * j + l] >> 4) | (((qh[l] >> (2 * j + 1)) & 1) << 4)) - m2;
    }
}

static void dec_q4_k(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b)), dmin = qxo_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *q = b + 16;
    for (int j = 0; j < 4; ++j) {
        uint8_t s, m;
        scale_min_k4(2 * j, sc, &s, &m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        scale_min_k4(2 * j + 1, sc, &s, &m);
        const float d2 = d * (float)s, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[64 * j + l] = d1 * (float)(q[32 * j + l] & 15) - m1;
        for (int l = 0; l < 32; ++l) y[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
    }
}

/* :2147-2169 */
static void dec_q6_k(const uint8_t *b, float *y) {
    const float d = qxo_fp16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; ++h) {
        const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[128 * h + l] = (d * (float)sc[is]) * (float)q1;
            y[128 * h + l + 32] = (d * (float)sc[is + 2]) * (float)q2;
            y[128 * h + l + 64] = (d * (float)sc[is + 4]) * (float)q3;
            y[128 * h + l + 96] = (d * (float)sc[is + 6]) * (float)q4;
        }
    }
}

static uint64_t block_bytes(uint32_t t) {
    switch (t) {
    case 12: return 144; case 13: return 176; case 14: return 210; case 17: return 74; case 18: return 98;
    case 21: return 110; case 22: return 82; case 23: return 136; default: return 0;
    }
}

/* :2195-2217 */
int qxo_decode_block(uint32_t t, const uint8_t *raw, float out[256]) {
    switch (t) {
    case 12: dec_q4_k(raw, out); return 1;
    case 14: dec_q6_k(raw, out); return 1;
    case 17: dec_iq2_xs(raw, out); return 1;
    case 18: dec_iq3_xxs(raw, out); return 1;
    case 13: dec_q5_k(raw, out); return 1;
    case 21: dec_iq3_s(raw, out); return 1;
    case 22: dec_iq2_s(raw, out); return 1;
    case 23: dec_iq4_xs(raw, out); return 1;
    default: return 0;
    }
}

/* ---- model file: minimal QXF1 directory view (reference include/qx_format.h:40-82) ---- */
struct qxo_model {
    int fd;
    uint64_t size;
    const uint8_t *map;
    uint32_t ntensors;
    const uint8_t *dir;
    uint32_t vocab, layers;
    int q8;   /* activation mode: 0 f32, 1 q8_k_compat */
};

qxo_model *qxo_open(const char *path) {
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 272) { close(fd); return NULL; }
    const uint8_t *map = (const uint8_t *)mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) { close(fd); return NULL; }
    if (memcmp(map, "QXF1", 4) != 0) { munmap((void *)map, (size_t)st.st_size); close(fd); return NULL; }
    qxo_model *m = (qxo_model *)calloc(1, sizeof(*m));
    m->fd = fd; m->size = (uint64_t)st.st_size; m->map = map;
    m->ntensors = rd32(map + 16);
    uint64_t dir_off;
    memcpy(&dir_off, map + 24, 8);
    m->dir = map + dir_off;
    m->layers = rd32(map + 56 + 8);
    m->vocab = rd32(map + 56 + 32);
    return m;
}

void qxo_close(qxo_model *m) {
    if (!m) return;
    munmap((void *)m->map, m->size);
    close(m->fd);
    free(m);
}

const uint8_t *qxo_tensor(const qxo_model *m, const char *name, uint32_t *type, uint64_t dims[4], uint64_t *bytes) {
    for (uint32_t i = 0; i < m->ntensors; ++i) {
        const uint8_t *e = m->dir + 208ull * i;
        if (strncmp((const char *)e, name, 96) == 0) {
            uint64_t off, sz;
            memcpy(&off, e + 144, 8);
            memcpy(&sz, e + 152, 8);
            if (type) *type = rd32(e + 164);
            if (dims) memcpy(dims, e + 112, 32);
            if (bytes) *bytes = sz;
            return m->map + off;
        }
    }
    return NULL;
}

static const uint8_t *tensor_l(const qxo_model *m, uint32_t layer, const char *suffix, uint32_t *type, uint64_t dims[4]) {
    char nm[96];
    snprintf(nm, sizeof(nm), "blk.%u.%s", layer, suffix);
    return qxo_tensor(m, nm, type, dims, NULL);
}

/* ---- primitives ---- */

/* :3358-3371 — double sum of squares, rms = sqrt(ss/n + 1e-6), y = (float)(x/rms) * w */
void qxo_rmsnorm(const float *x, const float *w, float *y, uint32_t n, double *rms_out) {
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const double rms = sqrt(ss / (double)n + 1.0e-6);
    for (uint32_t i = 0; i < n; ++i) y[i] = (float)((double)x[i] / rms) * w[i];
    if (rms_out) *rms_out = rms;
}

/* :3740-3757 — per-head, all in double */
void qxo_head_rmsnorm(float *v, const float *w, uint32_t heads, uint32_t hd) {
    for (uint32_t h = 0; h < heads; ++h) {
        float *p = v + (uint64_t)h * hd;
        double ss = 0.0;
        for (uint32_t d = 0; d < hd; ++d) ss += (double)p[d] * (double)p[d];
        const double inv = 1.0 / sqrt(ss / (double)hd + 1.0e-6);
        for (uint32_t d = 0; d < hd; ++d) p[d] = (float)((double)p[d] * inv * (double)w[d]);
    }
}

/* :4625-4641 — split-half pairs (i, i + hd/2) */
void qxo_rope(float *v, uint32_t heads, uint32_t hd, uint32_t pos, double theta) {
    const uint32_t half = hd / 2;
    for (uint32_t h = 0; h < heads; ++h) {
        float *p = v + (uint64_t)h * hd;
        for (uint32_t i = 0; i < half; ++i) {
            const double f = pow(theta, -(2.0 * (double)i) / (double)hd);
            const double a = (double)pos * f, c = cos(a), s = sin(a);
            const float x0 = p[i], x1 = p[i + half];
            p[i] = (float)((double)x0 * c - (double)x1 * s);
            p[i + half] = (float)((double)x0 * s + (double)x1 * c);
        }
    }
}

/* :4449-4463 */
float qxo_quantize_int8(const float *src, int8_t *dst, uint32_t n) {
    float mx = 0.0f;
    for (uint32_t i = 0; i < n; ++i) { float a = isfinite(src[i]) ? fabsf(src[i]) : 0.0f; if (a > mx) mx = a; }
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
    for (uint32_t i = 0; i < n; ++i) {
        int q = isfinite(src[i]) ? (int)lrintf(src[i] / scale) : 0;
        if (q < -127) q = -127;
        if (q > 127) q = 127;
        dst[i] = (int8_t)q;
    }
    return scale;
}

/* :4238-4291 (projections) and :4764-4784 (experts): per row, blocks in order,
 * acc += double(w_i) * double(x_i); store (float)acc, non-finite -> 0 */
static void matvec_f32(uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y,
                       double *probe) {
    const uint64_t bb = block_bytes(t), bpr = in_dims / 256u;
    float vals[256];
    double sum = 0.0;
    for (uint32_t r = 0; r < rows; ++r) {
        const uint8_t *row = w + (uint64_t)r * bpr * bb;
        double acc = 0.0;
        for (uint64_t b = 0; b < bpr; ++b) {
            qxo_decode_block(t, row + b * bb, vals);
            for (int i = 0; i < 256; ++i) acc += (double)vals[i] * (double)x[256 * b + i];
        }
        if (!isfinite(acc)) acc = 0.0;
        y[r] = (float)acc;
        sum += acc;   /* the probe: row dots before narrowing (:4276-4283) */
    }
    if (probe) *probe = sum;
}
void qxo_matvec(uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y) {
    matvec_f32(t, w, rows, in_dims, x, y, NULL);
}

/* ---- q8_k_compat activation mode (:3869-4205) ----
 * Activations become Q8_K blocks (ggml's block_q8_K layout: f32 d, 256 int8, 16 int16
 * sums); each weight type has an integer dot against them with float scaling per
 * block, in the reference's float op order. */

/* :3884-3889 — round half to even through the 1.5*2^23 bias (exact for |v| < 2^22) */
static int32_t q8_round(float v) {
    const float b = v + 12582912.0f;
    uint32_t u;
    memcpy(&u, &b, 4);
    return (int32_t)(u & 0x7fffffu) - 0x400000;
}

/* :3891-3927 — per 256 values: the value of largest magnitude (first on ties) maps
 * to -127; d = 1/(-127/max); codes clamp to [-128, 127]; 16 sums of 16 codes.
 * Returns 0 for a length that is not a multiple of 256 or a non-finite value. */
int qxo_quantize_q8k(const float *x, uint32_t n, qxo_q8k *out) {
    if (!n || n % 256u) return 0;
    for (uint32_t b = 0; b < n / 256u; ++b) {
        const float *v = x + 256ull * b;
        float amax = 0.0f, vmax = 0.0f;
        for (int i = 0; i < 256; ++i) {
            if (!isfinite(v[i])) return 0;
            if (fabsf(v[i]) > amax) { amax = fabsf(v[i]); vmax = v[i]; }
        }
        const float inv = vmax == 0.0f ? 0.0f : -127.0f / vmax;
        out[b].d = inv == 0.0f ? 0.0f : 1.0f / inv;
        for (int g = 0; g < 16; ++g) {
            int32_t sum = 0;
            for (int i = 16 * g; i < 16 * g + 16; ++i) {
                int32_t q = inv == 0.0f ? 0 : q8_round(inv * v[i]);
                q = q > 127 ? 127 : q < -128 ? -128 : q;
                out[b].qs[i] = (int8_t)q;
                sum += q;
            }
            out[b].bsums[g] = (int16_t)sum;
        }
    }
    return 1;
}

/* signed integer codes of the 32 values of sub-block ib (grid byte times sign) for the
 * codebook types; the block scales are applied by the callers */
static void iq_codes32(uint32_t t, const uint8_t *b, int ib, int32_t c[32]) {
    for (int l = 0; l < 4; ++l) {
        uint32_t idx[2] = {0, 0};
        uint8_t sg = 0;
        int per = 8;
        if (t == 17) {
            const uint16_t q = rd16(b + 2 + 2 * (4 * ib + l));
            idx[0] = q & 511u; sg = ksign(q >> 9);
        } else if (t == 22) {
            idx[0] = (uint32_t)b[2 + 4 * ib + l] | (((uint32_t)b[66 + ib] << (8 - 2 * l)) & 0x300u);
            sg = b[34 + 4 * ib + l];
        } else if (t == 18) {
            idx[0] = b[2 + 8 * ib + 2 * l]; idx[1] = b[2 + 8 * ib + 2 * l + 1];
            sg = ksign((rd32(b + 66 + 4 * ib) >> (7 * l)) & 127u); per = 4;
        } else {   /* 21 */
            const uint32_t qh = b[66 + ib];
            idx[0] = (uint32_t)b[2 + 8 * ib + 2 * l] | ((qh << (8 - 2 * l)) & 256u);
            idx[1] = (uint32_t)b[2 + 8 * ib + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256u);
            sg = b[74 + 4 * ib + l]; per = 4;
        }
        for (int j = 0; j < 8; ++j) {
            const uint32_t id = idx[j / per];
            const int jj = j % per;
            const int g = t == 17 ? iq2_grid_byte(id, jj) : t == 22 ? iq2s_grid_byte(id, jj)
                        : t == 18 ? iq3_grid_byte(id, jj) : iq3s_grid_byte(id, jj);
            c[8 * l + j] = (sg >> j) & 1 ? -g : g;
        }
    }
}

/* one row of nb blocks against nb Q8_K blocks:
 * IQ4_XS :3929-3952, Q5_K :3954-3986, Q6_K :3988-4021, IQ2_XS :4066-4099,
 * IQ2_S :4101-4133, IQ3_XXS :4135-4166, IQ3_S :4168-4205 */
static float dot_q8k(uint32_t t, const uint8_t *row, const qxo_q8k *a, uint32_t nb) {
    const uint64_t bb = block_bytes(t);
    if (t == 23) {
        float total = 0.0f;
        for (uint32_t k = 0; k < nb; ++k) {
            const uint8_t *b = row + k * bb;
            const float d = qxo_fp16_to_f32(rd16(b)) * a[k].d;
            const uint16_t sh = rd16(b + 2);
            for (int ib = 0; ib < 8; ++ib) {
                const int ls = ((b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
                int32_t dot = 0;
                for (int j = 0; j < 16; ++j) {
                    const uint8_t q = b[8 + 16 * ib + j];
                    dot += (int32_t)a[k].qs[32 * ib + j] * qx_iq4nl_values[q & 15];
                    dot += (int32_t)a[k].qs[32 * ib + 16 + j] * qx_iq4nl_values[q >> 4];
                }
                total += d * (float)(ls - 32) * (float)dot;
            }
        }
        return total;
    }
    if (t == 13) {
        float lanes[8] = {0}, sumf = 0.0f;
        for (uint32_t k = 0; k < nb; ++k) {
            const uint8_t *b = row + k * bb;
            const float d = qxo_fp16_to_f32(rd16(b)), dmin = qxo_fp16_to_f32(rd16(b + 2));
            int32_t li[8] = {0}, msum = 0;
            for (int g = 0; g < 8; ++g) {
                uint8_t sc, mn;
                scale_min_k4(g, b + 4, &sc, &mn);
                msum += ((int32_t)a[k].bsums[2 * g] + a[k].bsums[2 * g + 1]) * (int32_t)mn;
                for (int i = 0; i < 32; ++i) {
                    const uint8_t q = b[48 + 32 * (g / 2) + i];
                    const int32_t code = (g & 1 ? q >> 4 : q & 15) + (b[16 + i] >> g & 1 ? 16 : 0);
                    li[i & 7] += (int32_t)sc * code * a[k].qs[32 * g + i];
                }
            }
            const float sd = d * a[k].d;
            for (int l = 0; l < 8; ++l) lanes[l] += sd * (float)li[l];
            sumf -= dmin * a[k].d * (float)msum;
        }
        for (int l = 0; l < 8; ++l) sumf += lanes[l];
        return sumf;
    }
    if (t == 14) {
        float lanes[8] = {0};
        for (uint32_t k = 0; k < nb; ++k) {
            const uint8_t *b = row + k * bb;
            int32_t code[256];
            for (int h = 0; h < 2; ++h) {
                const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
                for (int i = 0; i < 32; ++i) {
                    code[128 * h + i] = ((ql[i] & 15) | ((qh[i] & 3) << 4)) - 32;
                    code[128 * h + i + 32] = ((ql[i + 32] & 15) | (((qh[i] >> 2) & 3) << 4)) - 32;
                    code[128 * h + i + 64] = ((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32;
                    code[128 * h + i + 96] = ((ql[i + 32] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32;
                }
            }
            int32_t li[8] = {0};
            for (int i = 0; i < 256; ++i) li[i & 7] += (int32_t)(int8_t)b[192 + i / 16] * a[k].qs[i] * code[i];
            const float d = qxo_fp16_to_f32(rd16(b + 208)) * a[k].d;
            for (int l = 0; l < 8; ++l) lanes[l] += d * (float)li[l];
        }
        float total = 0.0f;
        for (int l = 0; l < 8; ++l) total += lanes[l];
        return total;
    }
    /* codebook types: integer block sum, one float term per block */
    float sumf = 0.0f;
    for (uint32_t k = 0; k < nb; ++k) {
        const uint8_t *b = row + k * bb;
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            int32_t c[32], s0 = 0, s1 = 0;
            iq_codes32(t, b, ib, c);
            for (int i = 0; i < 16; ++i) s0 += c[i] * a[k].qs[32 * ib + i];
            for (int i = 16; i < 32; ++i) s1 += c[i] * a[k].qs[32 * ib + i];
            if (t == 17 || t == 22) {
                const uint8_t sc = t == 17 ? b[66 + ib] : b[74 + ib];
                bsum += s0 * (2 * (sc & 15) + 1) + s1 * (2 * (sc >> 4) + 1);
            } else if (t == 18) {
                bsum += (s0 + s1) * (int32_t)(2u * (rd32(b + 66 + 4 * ib) >> 28) + 1u);
            } else {
                bsum += (s0 + s1) * (2 * ((b[106 + ib / 2] >> (4 * (ib & 1))) & 15) + 1);
            }
        }
        sumf += qxo_fp16_to_f32(rd16(b)) * a[k].d * (float)bsum;
    }
    return t == 17 || t == 22 ? 0.125f * sumf : t == 18 ? 0.25f * sumf : sumf;
}

/* Q8_K matvec: the activation is quantized once (0 on a non-finite value, :3906).
 * Projections (:4257-4262) store a non-finite row as 0; expert rows (:4771) fail. */
static int matvec_q8k(uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y,
                      int expert) {
    qxo_q8k a[16];
    const uint32_t nb = in_dims / 256u;
    if (nb > 16 || !qxo_quantize_q8k(x, in_dims, a)) return 0;
    const uint64_t rb = nb * block_bytes(t);
    for (uint32_t r = 0; r < rows; ++r) {
        const float v = dot_q8k(t, w + r * rb, a, nb);
        if (!isfinite(v) && expert) return 0;
        y[r] = isfinite(v) ? v : 0.0f;
    }
    return 1;
}

void qxo_set_activation(qxo_model *m, int q8_k_compat) { m->q8 = q8_k_compat != 0; }

int qxo_matvec_q8k(uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y, int expert) {
    return block_bytes(t) ? matvec_q8k(t, w, rows, in_dims, x, y, expert) : 0;
}

/* attention projections: Q8_K for Q5_K / Q6_K / IQ4_XS in q8_k_compat mode (:4217-4218);
 * *probe (may be NULL) receives the sum of the rows' dots (:4276-4287) */
static int project_probe(const qxo_model *m, uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims,
                         const float *x, float *y, double *probe) {
    if (m->q8 && (t == 13 || t == 14 || t == 23)) {
        if (!matvec_q8k(t, w, rows, in_dims, x, y, 0)) return 0;
        if (probe) {
            double sum = 0.0;
            for (uint32_t r = 0; r < rows; ++r) sum += (double)y[r];
            *probe = sum;
        }
        return 1;
    }
    matvec_f32(t, w, rows, in_dims, x, y, probe);
    return 1;
}
static int project(const qxo_model *m, uint32_t t, const uint8_t *w, uint32_t rows, uint32_t in_dims,
                   const float *x, float *y) {
    return project_probe(m, t, w, rows, in_dims, x, y, NULL);
}

typedef struct { uint32_t token; double logit; } topent;

static void top_insert(topent *top, uint32_t n, uint32_t token, double logit) {
    for (uint32_t r = 0; r < n; ++r) {
        if (logit > top[r].logit) {
            for (uint32_t k = n - 1; k > r; --k) top[k] = top[k - 1];
            top[r].token = token; top[r].logit = logit;
            return;
        }
    }
}

/* :3554-3738 (f32 / baseline / serial): output_norm, then per row double dot,
 * non-finite -> error, float store, strict-> top-N insertion in row order */
int qxo_final_head(qxo_model *m, const float *residual, float *norm_out, float *logits,
                   uint32_t top_n, uint32_t *top_ids, double *top_logits) {
    uint32_t t;
    uint64_t dims[4];
    const float *nw = (const float *)qxo_tensor(m, "output_norm.weight", NULL, NULL, NULL);
    const uint8_t *W = qxo_tensor(m, "output.weight", &t, dims, NULL);
    if (!nw || !W || t != 14 || dims[0] != 2048) return 0;
    if (top_n == 0) top_n = 1;
    if (top_n > 32) top_n = 32;
    float xn[2048];
    qxo_rmsnorm(residual, nw, xn, 2048, NULL);
    if (norm_out) memcpy(norm_out, xn, sizeof(xn));
    topent top[32];
    for (uint32_t i = 0; i < top_n; ++i) { top[i].token = 0; top[i].logit = -1.0e300; }
    const uint32_t vocab = (uint32_t)dims[1];
    float vals[256];
    qxo_q8k a[8];
    if (m->q8 && !qxo_quantize_q8k(xn, 2048, a)) return 0;   /* :3666, 4026-4027 */
    for (uint32_t r = 0; r < vocab; ++r) {
        const uint8_t *row = W + (uint64_t)r * 8 * 210;
        double acc = 0.0;
        if (m->q8) {
            acc = (double)dot_q8k(14, row, a, 8);   /* :4039-4040 */
        } else {
            for (int b = 0; b < 8; ++b) {
                dec_q6_k(row + 210 * b, vals);
                for (int i = 0; i < 256; ++i) acc += (double)vals[i] * (double)xn[256 * b + i];
            }
        }
        if (!isfinite(acc)) return 0;
        if (logits) logits[r] = (float)acc;
        top_insert(top, top_n, r, acc);
    }
    for (uint32_t i = 0; i < top_n; ++i) {
        if (top_ids) top_ids[i] = top[i].token;
        if (top_logits) top_logits[i] = top[i].logit;
    }
    return 1;
}

static double silu(double x) { return x / (1.0 + exp(-x)); }   /* :2511-2513 */

/* :5198-5317 (f32) */
int qxo_moe_layer(qxo_model *m, uint32_t layer, const float *x, float *out, float *moe_out,
                  uint32_t ids[8], double wts[8]) {
    uint32_t tg, tu, td, tr;
    uint64_t dg[4], dr[4];
    const float *nw = (const float *)tensor_l(m, layer, "ffn_norm.weight", NULL, NULL);
    const float *R = (const float *)tensor_l(m, layer, "ffn_gate_inp.weight", &tr, dr);
    const uint8_t *G = tensor_l(m, layer, "ffn_gate_exps.weight", &tg, dg);
    const uint8_t *U = tensor_l(m, layer, "ffn_up_exps.weight", &tu, NULL);
    const uint8_t *D = tensor_l(m, layer, "ffn_down_exps.weight", &td, NULL);
    if (!nw || !R || !G || !U || !D || tr != 0) return 0;
    const uint32_t E = (uint32_t)dr[1], F = (uint32_t)dg[1];
    float xn[2048], moe[2048], g[768], u[768], h[768], y[2048];
    qxo_rmsnorm(x, nw, xn, 2048, NULL);
    double logit[128], p[128], mx = -1.0e300;
    for (uint32_t e = 0; e < E; ++e) {
        double acc = 0.0;
        for (uint32_t i = 0; i < 2048; ++i) acc += (double)R[(uint64_t)e * 2048 + i] * (double)xn[i];
        logit[e] = acc;
        if (acc > mx) mx = acc;
    }
    double den = 0.0;
    for (uint32_t e = 0; e < E; ++e) { p[e] = exp(logit[e] - mx); den += p[e]; }
    if (!isfinite(den) || den <= 0.0) return 0;
    for (uint32_t e = 0; e < E; ++e) p[e] /= den;
    uint8_t picked[128] = {0};
    double sel = 0.0;
    for (int r = 0; r < 8; ++r) {
        uint32_t best = 0;
        double bp = -1.0;
        for (uint32_t e = 0; e < E; ++e) if (!picked[e] && p[e] > bp) { best = e; bp = p[e]; }
        picked[best] = 1;
        ids[r] = best;
        wts[r] = bp;
        sel += bp;
    }
    if (!isfinite(sel) || sel <= 0.0) return 0;
    for (int r = 0; r < 8; ++r) wts[r] /= sel;
    memset(moe, 0, sizeof(moe));
    const uint64_t gate_expert = (uint64_t)F * 8 * block_bytes(tg), up_expert = (uint64_t)F * 8 * block_bytes(tu),
                   down_expert = 2048ull * (F / 256) * block_bytes(td);
    if (!gate_expert || !up_expert || !down_expert) return 0;
    /* q8_k_compat (:5286-5300): gate/up when both are IQ2_XS or both IQ2_S, down when
       IQ3_XXS, IQ3_S or IQ4_XS */
    const int gu_q8 = m->q8 && ((tg == 17 && tu == 17) || (tg == 22 && tu == 22));
    const int dn_q8 = m->q8 && (td == 18 || td == 21 || td == 23);
    for (int r = 0; r < 8; ++r) {
        if (gu_q8) {
            if (!matvec_q8k(tg, G + ids[r] * gate_expert, F, 2048, xn, g, 1) ||
                !matvec_q8k(tu, U + ids[r] * up_expert, F, 2048, xn, u, 1)) return 0;
        } else {
            qxo_matvec(tg, G + ids[r] * gate_expert, F, 2048, xn, g);
            qxo_matvec(tu, U + ids[r] * up_expert, F, 2048, xn, u);
        }
        for (uint32_t i = 0; i < F; ++i) h[i] = (float)(silu((double)g[i]) * (double)u[i]);
        if (dn_q8) {
            if (!matvec_q8k(td, D + ids[r] * down_expert, 2048, F, h, y, 1)) return 0;
        } else {
            qxo_matvec(td, D + ids[r] * down_expert, 2048, F, h, y);
        }
        for (uint32_t i = 0; i < 2048; ++i) moe[i] += (float)(wts[r] * (double)y[i]);
    }
    for (uint32_t i = 0; i < 2048; ++i) out[i] = x[i] + moe[i];
    if (moe_out) memcpy(moe_out, moe, sizeof(moe));
    return 1;
}

/* state loop :6282-6363 (norm, K/V, k norm, RoPE, INT8 store) then
 * qx_rope_gqa_attention_partial :5051-5196 */
int qxo_attention_layer(qxo_model *m, uint32_t layer, uint32_t pos, uint32_t ctx,
                        const float *x, int8_t *kc, int8_t *vc, float *ks, float *vs,
                        float *attn_out, float *kqv_out, float *vcur_out) {
    return qxo_attention_layer_ex(m, layer, pos, ctx, x, kc, vc, ks, vs, attn_out, kqv_out, vcur_out, 0, NULL, NULL, NULL);
}

/* The same, with the position's own INT8 K/V row and scales also written to row_k,
 * row_v (512 codes each) and row_scales (k, v) when given; with keep_row the cache's row
 * at [layer][pos] is left as the caller put it and attended to instead of the computed
 * one (a same-input replay of a device's attention on its own cache rows). */
int qxo_attention_layer_ex(qxo_model *m, uint32_t layer, uint32_t pos, uint32_t ctx,
                           const float *x, int8_t *kc, int8_t *vc, float *ks, float *vs,
                           float *attn_out, float *kqv_out, float *vcur_out,
                           int keep_row, int8_t *row_k, int8_t *row_v, float *row_scales) {
    uint32_t tq, tk, tv, to;
    const float *an = (const float *)tensor_l(m, layer, "attn_norm.weight", NULL, NULL);
    const uint8_t *Wq = tensor_l(m, layer, "attn_q.weight", &tq, NULL);
    const uint8_t *Wk = tensor_l(m, layer, "attn_k.weight", &tk, NULL);
    const uint8_t *Wv = tensor_l(m, layer, "attn_v.weight", &tv, NULL);
    const uint8_t *Wo = tensor_l(m, layer, "attn_output.weight", &to, NULL);
    const float *qn = (const float *)tensor_l(m, layer, "attn_q_norm.weight", NULL, NULL);
    const float *kn = (const float *)tensor_l(m, layer, "attn_k_norm.weight", NULL, NULL);
    if (!an || !Wq || !Wk || !Wv || !Wo || !qn || !kn || pos >= ctx) return 0;
    float xn[2048], k[512], v[512];
    float q[4096], cx[4096];
    qxo_rmsnorm(x, an, xn, 2048, NULL);
    if (!project(m, tk, Wk, 512, 2048, xn, k) || !project(m, tv, Wv, 512, 2048, xn, v)) return 0;
    qxo_head_rmsnorm(k, kn, 4, 128);
    qxo_rope(k, 4, 128, pos, 1000000.0);
    if (vcur_out) memcpy(vcur_out, v, sizeof(v));
    const uint64_t slot = (uint64_t)layer * ctx + pos;
    int8_t k8[512], v8[512];
    const float ksc = qxo_quantize_int8(k, k8, 512), vsc = qxo_quantize_int8(v, v8, 512);
    if (row_k) memcpy(row_k, k8, sizeof(k8));
    if (row_v) memcpy(row_v, v8, sizeof(v8));
    if (row_scales) { row_scales[0] = ksc; row_scales[1] = vsc; }
    if (!keep_row) {
        memcpy(kc + slot * 512, k8, sizeof(k8));
        memcpy(vc + slot * 512, v8, sizeof(v8));
        ks[slot] = ksc;
        vs[slot] = vsc;
    }
    if (!project(m, tq, Wq, 4096, 2048, xn, q)) return 0;
    qxo_head_rmsnorm(q, qn, 32, 128);
    qxo_rope(q, 32, 128, pos, 1000000.0);
    memset(cx, 0, sizeof(cx));
    const uint32_t n = pos + 1;
    double *sc = (double *)malloc(sizeof(double) * n);
    for (uint32_t qh = 0; qh < 32; ++qh) {
        const uint32_t kvh = qh / 8;
        double mx = -1e300;
        for (uint32_t t = 0; t < n; ++t) {
            const uint64_t sl = (uint64_t)layer * ctx + t;
            const int8_t *kp = kc + sl * 512 + kvh * 128;
            double s = 0.0;
            for (uint32_t d = 0; d < 128; ++d) s += (double)q[qh * 128 + d] * (double)((float)kp[d] * ks[sl]);
            s /= sqrt(128.0);
            if (!isfinite(s)) s = 0.0;
            sc[t] = s;
            if (s > mx) mx = s;
        }
        double den = 0.0;
        for (uint32_t t = 0; t < n; ++t) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
        if (!isfinite(den) || den <= 0.0) den = 1.0;
        for (uint32_t t = 0; t < n; ++t) {
            const double w = sc[t] / den;
            const uint64_t sl = (uint64_t)layer * ctx + t;
            const int8_t *vp = vc + sl * 512 + kvh * 128;
            for (uint32_t d = 0; d < 128; ++d) cx[qh * 128 + d] += (float)(w * (double)((float)vp[d] * vs[sl]));
        }
    }
    free(sc);
    if (kqv_out) memcpy(kqv_out, cx, sizeof(cx));
    return project(m, to, Wo, 2048, 4096, cx, attn_out);
}

/* :3759-3793 — the Q4_K row of `token`, no norm on the full-MoE path */
int qxo_embed(qxo_model *m, uint32_t token, float *x) {
    uint32_t t;
    uint64_t dims[4], bytes;
    const uint8_t *E = qxo_tensor(m, "token_embd.weight", &t, dims, &bytes);
    if (!E || t != 12 || token >= m->vocab) return 0;
    const uint64_t row = bytes / m->vocab;
    for (int b = 0; b < 8; ++b) dec_q4_k(E + token * row + 144ull * b, x + 256 * b);
    return 1;
}

/* state loop :6250-6627 for one --full-moe step */
int qxo_decode_token(qxo_model *m, uint32_t token, uint32_t pos, uint32_t ctx, uint32_t layers,
                     int8_t *kc, int8_t *vc, float *ks, float *vs,
                     float *residual_out, float *layer_out, int run_head, float *logits,
                     uint32_t top_n, uint32_t *top_ids, double *top_logits) {
    float x[2048], a[2048], y[2048];
    uint32_t ids[8];
    double w[8];
    if (!qxo_embed(m, token, x)) return 0;
    for (uint32_t l = 0; l < layers; ++l) {
        if (!qxo_attention_layer(m, l, pos, ctx, x, kc, vc, ks, vs, a, NULL, NULL)) return 0;
        for (int i = 0; i < 2048; ++i) x[i] += a[i];
        if (!qxo_moe_layer(m, l, x, y, NULL, ids, w)) return 0;
        memcpy(x, y, sizeof(x));
        if (layer_out) memcpy(layer_out + 2048ull * l, x, sizeof(x));
    }
    if (residual_out) memcpy(residual_out, x, sizeof(x));
    if (run_head) return qxo_final_head(m, x, NULL, logits, top_n, top_ids, top_logits);
    return 1;
}

/* :1878-1902 — f32 to IEEE binary16 with round-to-nearest-even, overflow to infinity,
 * NaN to a quiet NaN of the same sign (restated from the IEEE rules) */
uint16_t qxo_f32_to_fp16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t ex = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    if (ex == 0xffu) return (uint16_t)(sign | (man ? 0x7e00u : 0x7c00u));
    const int e16 = (int)ex - 112;   /* rebias 127 -> 15 */
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e16 <= 0) {                  /* binary16 subnormal (or zero): value / 2^-24, rounded */
        if (e16 < -10) return sign;
        const uint32_t full = man | 0x800000u, sh = (uint32_t)(14 - e16);
        uint32_t q = full >> sh;
        const uint32_t rem = full & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);   /* q == 0x400 carries into the smallest normal */
    }
    uint32_t q = ((uint32_t)e16 << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;   /* a carry can reach infinity */
    return (uint16_t)(sign | q);
}

/* attention stage probe (:5478-5586): one token attending to itself -- RMSNorm, V
 * projection, each q head's context is its kv head's v (softmax weight 1; an fp16
 * round trip with f16 KV), O projection, ffn_inp = x + O ctx.  probes: the V and O
 * projections' row-dot sums.  Returns 0 on a non-finite output (:5560-5564). */
int qxo_attention_stage(qxo_model *m, uint32_t layer, const float *x, int f16_kv, float *norm, float *vcur,
                        float *kqv, float *attn_out, float *ffn_inp, double probes[2]) {
    uint32_t tv, to;
    const float *an = (const float *)tensor_l(m, layer, "attn_norm.weight", NULL, NULL);
    const uint8_t *Wv = tensor_l(m, layer, "attn_v.weight", &tv, NULL);
    const uint8_t *Wo = tensor_l(m, layer, "attn_output.weight", &to, NULL);
    if (!an || !Wv || !Wo) return 0;
    qxo_rmsnorm(x, an, norm, 2048, NULL);
    if (!project_probe(m, tv, Wv, 512, 2048, norm, vcur, &probes[0])) return 0;
    for (uint32_t qh = 0; qh < 32; ++qh)
        for (uint32_t d = 0; d < 128; ++d) {
            const float v = vcur[(qh / 8) * 128 + d];
            kqv[qh * 128 + d] = f16_kv ? qxo_fp16_to_f32(qxo_f32_to_fp16(v)) : v;
        }
    if (!project_probe(m, to, Wo, 2048, 4096, kqv, attn_out, &probes[1])) return 0;
    for (uint32_t i = 0; i < 2048; ++i) {
        ffn_inp[i] = x[i] + attn_out[i];
        if (!isfinite(attn_out[i]) || !isfinite(ffn_inp[i])) return 0;
    }
    return 1;
}

/* MoE stage probe (:5588-5725): router logits narrowed to f32, f32 softmax
 * probabilities (exp of logit - max in double, normalised by their double sum), 8
 * picks by probability (strictly larger, lower index on ties), f32 weights renormalised
 * by their double sum, then per pick gate, up, SwiGLU, down and the weighted down
 * rows.  out: the QXO_MOE_STAGE block (see qxo.h). */
int qxo_moe_stage(qxo_model *m, uint32_t layer, const float *x, float *out, uint32_t ids[8]) {
    uint32_t tg, tu, td, tr;
    uint64_t dg[4], dr[4];
    const float *nw = (const float *)tensor_l(m, layer, "ffn_norm.weight", NULL, NULL);
    const float *R = (const float *)tensor_l(m, layer, "ffn_gate_inp.weight", &tr, dr);
    const uint8_t *G = tensor_l(m, layer, "ffn_gate_exps.weight", &tg, dg);
    const uint8_t *U = tensor_l(m, layer, "ffn_up_exps.weight", &tu, NULL);
    const uint8_t *D = tensor_l(m, layer, "ffn_down_exps.weight", &td, NULL);
    if (!nw || !R || !G || !U || !D || tr != 0) return 0;
    const uint32_t E = (uint32_t)dr[1], F = (uint32_t)dg[1];
    if (E < 8 || E > 128 || F != 768) return 0;
    float *norm = out, *logits = norm + 2048, *probs = logits + E, *topk = probs + E, *wts = topk + 8,
          *wsum = wts + 8, *wn = wsum + 1, *gate = wn + 8, *up = gate + 8 * 768, *sw = up + 8 * 768,
          *down = sw + 8 * 768, *weighted = down + 8 * 2048;
    qxo_rmsnorm(x, nw, norm, 2048, NULL);
    double mx = -1.0e300;
    for (uint32_t e = 0; e < E; ++e) {
        double acc = 0.0;
        for (uint32_t i = 0; i < 2048; ++i) acc += (double)R[(uint64_t)e * 2048 + i] * (double)norm[i];
        if (!isfinite(acc)) return 0;
        logits[e] = (float)acc;
        if (acc > mx) mx = acc;
    }
    double den = 0.0;
    for (uint32_t e = 0; e < E; ++e) { probs[e] = (float)exp((double)logits[e] - mx); den += probs[e]; }
    if (!isfinite(den) || den <= 0.0) return 0;
    for (uint32_t e = 0; e < E; ++e) probs[e] = (float)((double)probs[e] / den);
    uint8_t picked[128] = {0};
    double sum = 0.0;
    for (int r = 0; r < 8; ++r) {
        uint32_t best = 0;
        float bp = -1.0f;
        for (uint32_t e = 0; e < E; ++e) if (!picked[e] && probs[e] > bp) { best = e; bp = probs[e]; }
        picked[best] = 1;
        ids[r] = best;
        topk[r] = (float)best;
        wts[r] = bp;
        sum += bp;
    }
    if (!isfinite(sum) || sum <= 0.0) return 0;
    wsum[0] = (float)sum;
    for (int r = 0; r < 8; ++r) wn[r] = (float)((double)wts[r] / sum);
    const uint64_t gate_expert = (uint64_t)F * 8 * block_bytes(tg), up_expert = (uint64_t)F * 8 * block_bytes(tu),
                   down_expert = 2048ull * (F / 256) * block_bytes(td);
    const int gu_q8 = m->q8 && ((tg == 17 && tu == 17) || (tg == 22 && tu == 22));
    const int dn_q8 = m->q8 && (td == 18 || td == 21 || td == 23);
    for (int r = 0; r < 8; ++r) {
        float *g = gate + r * 768, *u = up + r * 768, *h = sw + r * 768, *y = down + r * 2048;
        if (gu_q8) {
            if (!matvec_q8k(tg, G + ids[r] * gate_expert, F, 2048, norm, g, 1) ||
                !matvec_q8k(tu, U + ids[r] * up_expert, F, 2048, norm, u, 1)) return 0;
        } else {
            qxo_matvec(tg, G + ids[r] * gate_expert, F, 2048, norm, g);
            qxo_matvec(tu, U + ids[r] * up_expert, F, 2048, norm, u);
        }
        for (uint32_t i = 0; i < F; ++i) h[i] = (float)(silu((double)g[i]) * (double)u[i]);
        if (dn_q8) {
            if (!matvec_q8k(td, D + ids[r] * down_expert, 2048, F, h, y, 1)) return 0;
        } else {
            qxo_matvec(td, D + ids[r] * down_expert, 2048, F, h, y);
        }
        for (uint32_t i = 0; i < 2048; ++i) weighted[r * 2048 + i] = (float)((double)y[i] * (double)wn[r]);
    }
    return 1;
}
