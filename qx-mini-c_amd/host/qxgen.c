/* Seeded random-init QXF1 writer for the Qwen3-30B-A3B-shaped model.
 *
 * Layout and tensor set follow the reference's QXF1 tensor-copy format
 * (reference include/qx_format.h:40-82; per-layer names src/qx_format.c:5208-5214,
 * 6283-6306, 3608-3609, 3761).  Content is random with these distributions, one
 * independent counter-seeded stream per 256-value block (so any tensor's bytes
 * depend only on (seed, tensor name), not on which other tensors are written):
 *   Q4_K  token_embd  : d, dmin = fp16(U[1e-3,4e-3]); scales, qs uniform bytes
 *   Q6_K  output      : ql, qh uniform bytes; scales int8 U[-32,31]; d = fp16(U[1e-4,1e-3])
 *   IQ4_XS attn q/k/v/o: d = fp16(U[1e-5,3e-5]); scales_h, scales_l, qs uniform
 *   IQ2_XS gate/up    : d = fp16(U[2e-4,5e-4]); qs (9-bit grid, 7-bit sign) and scales uniform
 *   IQ3_XXS down      : d = fp16(U[1e-4,3e-4]); qs bytes and aux32 words uniform
 * and, in the real-checkpoint mix (spec->mix = 1):
 *   Q5_K  attn v/o    : d, dmin = fp16(U[1e-5,3e-5]); scales, qh, qs uniform bytes
 *   IQ2_S gate/up     : d = fp16(U[2e-4,5e-4]); qs, signs, qh, scales uniform
 *   IQ3_S down        : d = fp16(U[1e-4,3e-4]); qs, qh, signs, scales uniform
 *   IQ4_XS down       : as the attention IQ4_XS
 *   F32 norms         : U(0.5,1.5);  router ffn_gate_inp: N(0, 0.02)
 * The fp16 ranges keep every projection output O(1) over 48 layers. */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "qx_host.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static void set_err(char *err, uint64_t n, const char *msg) {
    if (err && n) snprintf(err, (size_t)n, "%s", msg);
}

static uint64_t splitmix(uint64_t *s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static double unif(uint64_t *s) { return (double)(splitmix(s) >> 11) * (1.0 / 9007199254740992.0); }

/* round-to-nearest-even f32 -> fp16 bits (normal and subnormal ranges) */
static uint16_t f32_to_fp16(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t e = (b >> 23) & 0xffu, m = b & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0));
    int he = (int)e - 127 + 15;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        m |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - he);
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = m >> 13, rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    if (r == 0x400u) { r = 0; ++he; if (he >= 31) return (uint16_t)(sign | 0x7c00u); }
    return (uint16_t)(sign | ((uint32_t)he << 10) | r);
}

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static void fill_bytes(uint8_t *p, size_t n, uint64_t *s) {
    while (n >= 8) { uint64_t r = splitmix(s); memcpy(p, &r, 8); p += 8; n -= 8; }
    if (n) { uint64_t r = splitmix(s); memcpy(p, &r, n); }
}

static uint16_t fp16_unif(uint64_t *s, double lo, double hi) {
    return f32_to_fp16((float)(lo + (hi - lo) * unif(s)));
}

enum { DIST_NORM_W = 1, DIST_ROUTER = 2 };

typedef struct gen_tensor {
    char name[QXF_NAME_MAX];
    uint32_t type, rank, dist;
    uint64_t dims[4];
    uint64_t offset, bytes, blocks, block_bytes;
    uint64_t key;
    /* planted outliers (spec->outliers): F32 norms by channel (1: x1000 at channel 5 mod 128,
       2: also x1e6 at channel 1001); quantized rows: blocks of row out_row mod out_rows get
       their fp16 d range x1000 (0: none), bpr blocks per row */
    uint32_t out_norm;
    uint64_t out_rows, out_row, bpr;
    /* spec->outliers 3: the marked row's blocks get an exponent-31 fp16 d instead of x1000 */
    uint32_t sat;
} gen_tensor;

static int in_marked_row(const gen_tensor *t, uint64_t blk) {
    return t->out_rows && (blk / t->bpr) % t->out_rows == t->out_row;
}

/* fp16 d range factor of block blk: x1000 in a planted outlier row */
static double d_scale(const gen_tensor *t, uint64_t blk) {
    return !t->sat && in_marked_row(t, blk) ? 1000.0 : 1.0;
}

/* exponent-31 halves (+inf, -inf, NaN, NaN with the sign bit), taken in turn by block */
static const uint16_t SAT_D[4] = {0x7c00u, 0xfc00u, 0x7e00u, 0xfe01u};

/* one 256-value block (or 256 floats for F32) */
static void gen_block(const gen_tensor *t, uint64_t blk, uint8_t *out, uint64_t nbytes) {
    uint64_t s = t->key ^ (blk * 0xd1342543de82ef95ull);
    splitmix(&s);
    const double ds = d_scale(t, blk);
    switch (t->type) {
    case QXT_F32: {
        uint64_t n = nbytes / 4;
        for (uint64_t i = 0; i < n; ++i) {
            float v;
            if (t->dist == DIST_ROUTER) {
                double u1 = unif(&s), u2 = unif(&s);
                if (u1 < 1e-300) u1 = 1e-300;
                v = (float)(0.02 * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
            } else {
                v = (float)(0.5 + unif(&s));
                const uint64_t ch = blk * 256 + i;
                if (t->out_norm && ch % 128 == 5) v *= 1000.0f;
                if (t->out_norm == 2 && ch == 1001) v *= 1.0e6f;
            }
            memcpy(out + 4 * i, &v, 4);
        }
        break;
    }
    case QXT_Q4_K:
        put16(out, fp16_unif(&s, 1e-3, 4e-3));
        put16(out + 2, fp16_unif(&s, 1e-3, 4e-3));
        fill_bytes(out + 4, 140, &s);
        break;
    case QXT_Q6_K:
        fill_bytes(out, 192, &s);
        for (int i = 0; i < 16; ++i) out[192 + i] = (uint8_t)(int8_t)((int)(splitmix(&s) % 64u) - 32);
        put16(out + 208, fp16_unif(&s, 1e-4, 1e-3));
        break;
    case QXT_IQ4_XS:
        put16(out, fp16_unif(&s, 1e-5 * ds, 3e-5 * ds));
        fill_bytes(out + 2, 134, &s);
        break;
    case QXT_IQ2_XS:
        put16(out, fp16_unif(&s, 2e-4 * ds, 5e-4 * ds));
        fill_bytes(out + 2, 72, &s);
        break;
    case QXT_IQ3_XXS:
        put16(out, fp16_unif(&s, 1e-4 * ds, 3e-4 * ds));
        fill_bytes(out + 2, 96, &s);
        break;
    case QXT_Q5_K:
        put16(out, fp16_unif(&s, 1e-5 * ds, 3e-5 * ds));
        put16(out + 2, fp16_unif(&s, 1e-5, 3e-5));
        fill_bytes(out + 4, 172, &s);
        break;
    case QXT_IQ2_S:
        put16(out, fp16_unif(&s, 2e-4 * ds, 5e-4 * ds));
        fill_bytes(out + 2, 80, &s);
        break;
    case QXT_IQ3_S:
        put16(out, fp16_unif(&s, 1e-4 * ds, 3e-4 * ds));
        fill_bytes(out + 2, 108, &s);
        break;
    default:
        memset(out, 0, nbytes);
    }
    /* every quantized type but Q4_K / Q6_K leads with its fp16 d */
    if (t->sat && in_marked_row(t, blk) && t->type != QXT_F32 && t->type != QXT_Q4_K && t->type != QXT_Q6_K)
        put16(out, SAT_D[blk % 4]);
}

typedef struct gen_job {
    gen_tensor *t;
    uint32_t nt;
    uint8_t *base;
    atomic_uint_fast64_t next_chunk;
    uint64_t total_chunks;
    uint64_t *chunk_start;   /* prefix sums of per-tensor chunk counts */
    atomic_uint next_fnv;
    uint64_t *checksums;
} gen_job;

#define CHUNK_BLOCKS 4096ull

static void *gen_worker(void *arg) {
    gen_job *j = (gen_job *)arg;
    for (;;) {
        uint64_t c = atomic_fetch_add(&j->next_chunk, 1);
        if (c >= j->total_chunks) break;
        uint32_t ti = 0;
        while (ti + 1 < j->nt && j->chunk_start[ti + 1] <= c) ++ti;
        const gen_tensor *t = &j->t[ti];
        uint64_t b0 = (c - j->chunk_start[ti]) * CHUNK_BLOCKS;
        uint64_t b1 = b0 + CHUNK_BLOCKS < t->blocks ? b0 + CHUNK_BLOCKS : t->blocks;
        for (uint64_t b = b0; b < b1; ++b) {
            uint64_t off = b * t->block_bytes;
            uint64_t n = t->block_bytes;
            if (off + n > t->bytes) n = t->bytes - off;
            gen_block(t, b, j->base + t->offset + off, n);
        }
    }
    return NULL;
}

static void *fnv_worker(void *arg) {
    gen_job *j = (gen_job *)arg;
    for (;;) {
        unsigned i = atomic_fetch_add(&j->next_fnv, 1);
        if (i >= j->nt) break;
        j->checksums[i] = qxf_fnv1a64(j->base + j->t[i].offset, j->t[i].bytes);
    }
    return NULL;
}

static void add_tensor(gen_tensor *v, uint32_t *n, const char *name, uint32_t type, uint32_t rank,
                       uint64_t d0, uint64_t d1, uint64_t d2, uint32_t dist, uint64_t seed) {
    gen_tensor *t = &v[(*n)++];
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->type = type; t->rank = rank; t->dist = dist;
    t->dims[0] = d0; t->dims[1] = rank > 1 ? d1 : 0; t->dims[2] = rank > 2 ? d2 : 0;
    uint64_t elems = d0 * (rank > 1 ? d1 : 1) * (rank > 2 ? d2 : 1);
    uint64_t bv = 1, bb = 4;
    qxf_type_block(type, &bv, &bb);
    t->bytes = elems / bv * bb;
    if (type == QXT_F32) { t->block_bytes = 1024; t->blocks = (t->bytes + 1023) / 1024; }
    else { t->block_bytes = bb; t->blocks = elems / bv; }
    uint64_t k = seed ^ qxf_fnv1a64(name, strlen(name));
    splitmix(&k);
    t->key = k;
}

/* planted outliers of the last tensor added (spec->outliers) */
static void mark_norm(gen_tensor *t, uint32_t kind) { t->out_norm = kind; }
static void mark_rows(gen_tensor *t, uint64_t rows, uint64_t row) {
    t->out_rows = rows;
    t->out_row = row;
    t->bpr = t->dims[0] / 256;
}
static void mark_sat(gen_tensor *t, uint64_t rows, uint64_t row) {
    mark_rows(t, rows, row);
    t->sat = 1;
}

static uint32_t build_tensor_list(const qxgen_spec *sp, gen_tensor *v) {
    uint32_t n = 0;
    char nm[QXF_NAME_MAX];
    const int ol = sp->outliers == 1 || sp->outliers == 2, ol2 = sp->outliers == 2, sat = sp->outliers == 3;
    const uint64_t H = 2048, V = sp->vocab, E = sp->experts, F = 768;
    if (sp->with_embedding) add_tensor(v, &n, "token_embd.weight", QXT_Q4_K, 2, H, V, 0, 0, sp->seed);
    if (sp->with_head) {
        add_tensor(v, &n, "output_norm.weight", QXT_F32, 1, H, 0, 0, DIST_NORM_W, sp->seed);
        if (ol) mark_norm(&v[n - 1], ol2 ? 2 : 1);
        add_tensor(v, &n, "output.weight", QXT_Q6_K, 2, H, V, 0, 0, sp->seed);
    }
    for (uint32_t l = 0; l < sp->layers; ++l) {
#define T(suffix, ...) do { snprintf(nm, sizeof(nm), "blk.%u." suffix, l); add_tensor(v, &n, nm, __VA_ARGS__, sp->seed); } while (0)
        T("attn_norm.weight", QXT_F32, 1, H, 0, 0, DIST_NORM_W);
        if (ol) mark_norm(&v[n - 1], ol2 ? 2 : 1);
        T("attn_q.weight", QXT_IQ4_XS, 2, H, 4096, 0, 0);
        if (sat) mark_sat(&v[n - 1], 4096, 100);
        T("attn_k.weight", QXT_IQ4_XS, 2, H, 512, 0, 0);
        if (sat) mark_sat(&v[n - 1], 512, 7);
        const uint32_t k4 = sp->mix ? l % 4 : 0;
        const uint32_t t_vo = (k4 == 1 || k4 == 3) ? QXT_Q5_K : QXT_IQ4_XS;
        const uint32_t t_gu = (k4 == 1 || k4 == 3) ? QXT_IQ2_S : QXT_IQ2_XS;
        const uint32_t t_dn = k4 == 0 ? QXT_IQ3_XXS : k4 == 1 ? QXT_IQ4_XS : QXT_IQ3_S;
        T("attn_v.weight", t_vo, 2, H, 512, 0, 0);
        if (ol) mark_rows(&v[n - 1], 128, 3);
        if (sat) mark_sat(&v[n - 1], 512, 3);
        T("attn_output.weight", t_vo, 2, 4096, H, 0, 0);
        if (ol) mark_rows(&v[n - 1], H, 11);
        if (sat) mark_sat(&v[n - 1], H, 11);
        T("attn_q_norm.weight", QXT_F32, 1, 128, 0, 0, DIST_NORM_W);
        if (ol) mark_norm(&v[n - 1], 1);
        T("attn_k_norm.weight", QXT_F32, 1, 128, 0, 0, DIST_NORM_W);
        if (ol) mark_norm(&v[n - 1], 1);
        T("ffn_norm.weight", QXT_F32, 1, H, 0, 0, DIST_NORM_W);
        if (ol) mark_norm(&v[n - 1], 1);
        T("ffn_gate_inp.weight", QXT_F32, 2, H, E, 0, DIST_ROUTER);
        T("ffn_gate_exps.weight", t_gu, 3, H, F, E, 0);
        if (ol2) mark_rows(&v[n - 1], F, 7);
        if (sat) mark_sat(&v[n - 1], F, 7);
        T("ffn_up_exps.weight", t_gu, 3, H, F, E, 0);
        if (sat) mark_sat(&v[n - 1], F, 9);
        T("ffn_down_exps.weight", t_dn, 3, F, H, E, 0);
        if (ol2) mark_rows(&v[n - 1], H, 13);
        if (sat) mark_sat(&v[n - 1], H, 13);
#undef T
    }
    return n;
}

static uint32_t dtype_for(uint32_t type) {
    switch (type) {
    case QXT_F32: return 2;
    case QXT_IQ2_XS: case QXT_IQ2_S: return 5;
    case QXT_IQ3_XXS: case QXT_IQ3_S: return 4;
    default: return 3;
    }
}

static int write_fd(int fd, const qxgen_spec *spec, uint64_t *size_out, char *err, uint64_t err_len) {
    if (!spec || spec->layers > 48 || spec->experts < 8 || spec->experts > 128 || !spec->vocab || spec->outliers > 3 ||
        (!spec->layers && !spec->with_head && !spec->with_embedding)) {
        set_err(err, err_len, "invalid generator spec"); return 0;
    }
    uint32_t cap = 3 + 12 * spec->layers;
    gen_tensor *t = (gen_tensor *)calloc(cap, sizeof(gen_tensor));
    if (!t) { set_err(err, err_len, "out of memory"); return 0; }
    uint32_t nt = build_tensor_list(spec, t);
    uint64_t dir_off = QXF_ALIGN;
    uint64_t data_off = (dir_off + (uint64_t)nt * sizeof(qxf_dir_entry) + QXF_ALIGN - 1) / QXF_ALIGN * QXF_ALIGN;
    uint64_t off = data_off;
    for (uint32_t i = 0; i < nt; ++i) {
        t[i].offset = off;
        off = (off + t[i].bytes + QXF_ALIGN - 1) / QXF_ALIGN * QXF_ALIGN;
    }
    /* the last tensor ends the file exactly (no trailing pad needed by the reader,
       but keep the file size a multiple of the alignment like every offset) */
    uint64_t fsize = off;
    if (ftruncate(fd, (off_t)fsize) != 0) { free(t); set_err(err, err_len, strerror(errno)); return 0; }
    uint8_t *base = (uint8_t *)mmap(NULL, fsize, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (base == MAP_FAILED) { free(t); set_err(err, err_len, "mmap of output failed"); return 0; }

    gen_job job;
    memset(&job, 0, sizeof(job));
    job.t = t; job.nt = nt; job.base = base;
    job.chunk_start = (uint64_t *)calloc(nt + 1, sizeof(uint64_t));
    job.checksums = (uint64_t *)calloc(nt, sizeof(uint64_t));
    for (uint32_t i = 0; i < nt; ++i) job.chunk_start[i + 1] = job.chunk_start[i] + (t[i].blocks + CHUNK_BLOCKS - 1) / CHUNK_BLOCKS;
    job.total_chunks = job.chunk_start[nt];
    atomic_init(&job.next_chunk, 0);
    atomic_init(&job.next_fnv, 0);
    long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    uint32_t nth = spec->threads ? spec->threads : (uint32_t)(ncpu > 16 ? 16 : ncpu < 1 ? 1 : ncpu);
    pthread_t th[64];
    if (nth > 64) nth = 64;
    for (uint32_t i = 0; i < nth; ++i) pthread_create(&th[i], NULL, gen_worker, &job);
    for (uint32_t i = 0; i < nth; ++i) pthread_join(th[i], NULL);
    for (uint32_t i = 0; i < nth; ++i) pthread_create(&th[i], NULL, fnv_worker, &job);
    for (uint32_t i = 0; i < nth; ++i) pthread_join(th[i], NULL);

    qxf_header h;
    memset(&h, 0, sizeof(h));
    memcpy(h.magic, QXF_MAGIC, 4);
    h.version = QXF_VERSION;
    h.header_size = sizeof(qxf_header);
    h.dir_entry_size = sizeof(qxf_dir_entry);
    h.tensor_count = nt;
    h.dir_offset = dir_off;
    h.data_offset = data_off;
    h.file_size = fsize;
    qxf_manifest *m = &h.manifest;
    m->model_type = 2; m->quant_type = 4; m->layers = spec->layers ? spec->layers : 48;
    m->hidden = 2048; m->intermediate = 6144; m->q_heads = 32; m->kv_heads = 4; m->head_dim = 128;
    m->vocab = spec->vocab; m->max_ctx = 4096; m->experts = spec->experts; m->experts_per_token = 8;
    m->moe_intermediate = 768;
    h.manifest_checksum = qxf_fnv1a64(m, sizeof(*m));
    memcpy(base, &h, sizeof(h));
    qxf_dir_entry *dir = (qxf_dir_entry *)(base + dir_off);
    for (uint32_t i = 0; i < nt; ++i) {
        qxf_dir_entry *d = &dir[i];
        memset(d, 0, sizeof(*d));
        memcpy(d->name, t[i].name, QXF_NAME_MAX);
        d->dtype = dtype_for(t[i].type);
        d->quant = 4;
        d->rank = t[i].rank;
        for (int k = 0; k < 4; ++k) d->dims[k] = t[i].dims[k];
        d->offset = t[i].offset;
        d->byte_size = t[i].bytes;
        d->group_size = t[i].type == QXT_F32 ? 0 : 64;
        d->flags = t[i].type;
        d->checksum = job.checksums[i];
    }
    munmap(base, fsize);
    free(job.chunk_start);
    free(job.checksums);
    free(t);
    if (size_out) *size_out = fsize;
    return 1;
}

int qxgen_write(const char *path, const qxgen_spec *spec, uint64_t *file_size, char *err, uint64_t err_len) {
    if (!path) { set_err(err, err_len, "invalid argument"); return 0; }
    int fd = open(path, O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd < 0) { set_err(err, err_len, strerror(errno)); return 0; }
    int ok = write_fd(fd, spec, file_size, err, err_len);
    if (close(fd) != 0) ok = 0;
    if (!ok) unlink(path);
    return ok;
}

int qxgen_memfd(const qxgen_spec *spec, char *path_out, uint64_t path_len, int *fd_out, char *err, uint64_t err_len) {
    int fd = memfd_create("qxf-model", MFD_CLOEXEC);
    if (fd < 0) { set_err(err, err_len, strerror(errno)); return 0; }
    if (!write_fd(fd, spec, NULL, err, err_len)) { close(fd); return 0; }
    if (path_out) snprintf(path_out, (size_t)path_len, "/proc/self/fd/%d", fd);
    if (fd_out) *fd_out = fd;
    return 1;
}

void qxgen_memfd_close(int fd) { if (fd >= 0) close(fd); }
