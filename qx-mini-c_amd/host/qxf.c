/* QXF1 reader: validation rules of the reference loader (src/qx_format.c:438-460,
 * 652-841 of the reference), mmap-only (the GPU build uploads every tensor once,
 * so the buffered per-call read path has no use here). */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "qx_host.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

_Static_assert(sizeof(qxf_header) == 272, "QXF1 header is 272 bytes");
_Static_assert(sizeof(qxf_dir_entry) == 208, "QXF1 directory entry is 208 bytes");

static void set_err(char *err, uint64_t n, const char *msg) {
    if (err && n) snprintf(err, (size_t)n, "%s", msg);
}

uint64_t qxf_fnv1a64_update(uint64_t h, const void *data, uint64_t len) {
    const uint8_t *p = (const uint8_t *)data;
    for (uint64_t i = 0; i < len; ++i) { h ^= p[i]; h *= 1099511628211ull; }
    return h;
}

uint64_t qxf_fnv1a64(const void *data, uint64_t len) {
    return qxf_fnv1a64_update(1469598103934665603ull, data, len);
}

/* block geometry per ggml type: reference src/qx_format.c:667-691 */
int qxf_type_block(uint32_t t, uint64_t *bv, uint64_t *bb) {
    uint64_t v = 256, b = 0;
    switch (t) {
    case QXT_F32: v = 1; b = 4; break;
    case 1: v = 1; b = 2; break;          /* F16 */
    case 8: v = 32; b = 34; break;        /* Q8_0 */
    case 10: b = 84; break;               /* Q2_K */
    case 11: b = 110; break;              /* Q3_K */
    case QXT_Q4_K: b = 144; break;
    case QXT_Q5_K: b = 176; break;
    case QXT_Q6_K: b = 210; break;
    case QXT_IQ2_XS: b = 74; break;
    case QXT_IQ3_XXS: b = 98; break;
    case QXT_IQ3_S: b = 110; break;
    case QXT_IQ2_S: b = 82; break;
    case QXT_IQ4_XS: b = 136; break;
    default: return 0;
    }
    if (bv) *bv = v;
    if (bb) *bb = b;
    return 1;
}

/* dtype / group-size traits: reference src/qx_format.c:693-709 */
static int traits_ok(const qxf_dir_entry *t) {
    uint32_t dt = 0, grp = 0;
    switch (t->flags) {
    case 0: dt = 2; break;
    case 1: dt = 1; break;
    case 8: dt = 6; break;
    case 10: case 17: case 22: dt = 5; grp = 64; break;
    case 11: case 18: case 21: dt = 4; grp = 64; break;
    case 12: case 13: case 14: dt = 3; grp = 64; break;
    case 23: return (t->dtype == 3 && t->group_size == 64) || (t->dtype == 6 && t->group_size == 0);
    default: return 0;
    }
    return t->dtype == dt && t->group_size == grp;
}

static int manifest_ok(const qxf_manifest *m) {
    if (m->model_type != 1 && m->model_type != 2) return 0;
    if (m->quant_type < 1 || m->quant_type > 5) return 0;
    if (!m->layers || !m->hidden || !m->intermediate || !m->q_heads || !m->kv_heads ||
        m->kv_heads > m->q_heads || !m->head_dim || !m->vocab || !m->max_ctx) return 0;
    if (m->model_type == 2 && (!m->experts || !m->experts_per_token ||
        m->experts_per_token > m->experts || !m->moe_intermediate)) return 0;
    return 1;
}

typedef struct { uint64_t off, end; } span_t;

static int cmp_span(const void *a, const void *b) {
    const span_t *x = (const span_t *)a, *y = (const span_t *)b;
    return x->off < y->off ? -1 : x->off > y->off ? 1 : 0;
}

static int cmp_name(const void *a, const void *b) {
    return strcmp(*(const char *const *)a, *(const char *const *)b);
}

void qxf_close(qxf_file *f) {
    if (!f) return;
    if (f->map && f->map != MAP_FAILED) munmap((void *)f->map, (size_t)f->header.file_size);
    if (f->fd >= 0) close(f->fd);
    free(f->dir);
    memset(f, 0, sizeof(*f));
    f->fd = -1;
}

int qxf_open(const char *path, qxf_file *out, char *err, uint64_t err_len) {
    if (!path || !out) { set_err(err, err_len, "invalid argument"); return 0; }
    memset(out, 0, sizeof(*out));
    out->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (out->fd < 0) { set_err(err, err_len, strerror(errno)); return 0; }
    qxf_header *h = &out->header;
    if (pread(out->fd, h, sizeof(*h), 0) != (ssize_t)sizeof(*h)) { set_err(err, err_len, "short read header"); goto fail; }
    if (memcmp(h->magic, QXF_MAGIC, 4) != 0) { set_err(err, err_len, "bad QXF magic"); goto fail; }
    if (h->version != QXF_VERSION) { set_err(err, err_len, "unsupported QXF version"); goto fail; }
    if (h->header_size != sizeof(qxf_header) || h->dir_entry_size != sizeof(qxf_dir_entry)) {
        set_err(err, err_len, "QXF struct size mismatch"); goto fail;
    }
    if (qxf_fnv1a64(&h->manifest, sizeof(h->manifest)) != h->manifest_checksum) {
        set_err(err, err_len, "manifest checksum mismatch"); goto fail;
    }
    if (!manifest_ok(&h->manifest)) { set_err(err, err_len, "invalid QXF manifest"); goto fail; }
    if (h->tensor_count == 0) { set_err(err, err_len, "empty tensor directory"); goto fail; }
    struct stat st;
    if (fstat(out->fd, &st) != 0 || (uint64_t)st.st_size != h->file_size || h->file_size < sizeof(*h)) {
        set_err(err, err_len, "declared QXF file size does not match file"); goto fail;
    }
    uint64_t dir_bytes = (uint64_t)h->tensor_count * sizeof(qxf_dir_entry);
    if (h->dir_offset < h->header_size || h->dir_offset % QXF_ALIGN || h->data_offset % QXF_ALIGN ||
        h->dir_offset > h->file_size || dir_bytes > h->file_size - h->dir_offset ||
        h->data_offset < h->dir_offset + dir_bytes || h->data_offset > h->file_size) {
        set_err(err, err_len, "invalid QXF layout"); goto fail;
    }
    out->dir = (qxf_dir_entry *)calloc(h->tensor_count, sizeof(qxf_dir_entry));
    if (!out->dir) { set_err(err, err_len, "out of memory"); goto fail; }
    if (pread(out->fd, out->dir, dir_bytes, (off_t)h->dir_offset) != (ssize_t)dir_bytes) {
        set_err(err, err_len, "short tensor directory read"); goto fail;
    }
    {
        int meta_only = h->file_size == h->data_offset;
        const char **names = (const char **)malloc(h->tensor_count * sizeof(*names));
        span_t *spans = (span_t *)malloc(h->tensor_count * sizeof(*spans));
        if (!names || !spans) { free(names); free(spans); set_err(err, err_len, "out of memory"); goto fail; }
        const char *bad = NULL;
        for (uint32_t i = 0; i < h->tensor_count && !bad; ++i) {
            const qxf_dir_entry *t = &out->dir[i];
            if (!memchr(t->name, 0, QXF_NAME_MAX) || !t->name[0]) { bad = "unterminated or empty tensor name"; break; }
            names[i] = t->name;
            if (t->dtype < 1 || t->dtype > 6 || t->quant < 1 || t->quant > 5 || (!meta_only && !traits_ok(t))) {
                bad = "invalid tensor metadata"; break;
            }
            uint64_t elems = 1;
            if (t->rank == 0 || t->rank > QXF_MAX_DIMS) { bad = "invalid tensor dimensions"; break; }
            for (uint32_t d = 0; d < QXF_MAX_DIMS; ++d) {
                if (d < t->rank) {
                    if (!t->dims[d] || elems > UINT64_MAX / t->dims[d]) { bad = "invalid tensor dimensions"; break; }
                    elems *= t->dims[d];
                } else if (t->dims[d]) { bad = "invalid tensor dimensions"; break; }
            }
            if (bad) break;
            if (meta_only) {
                if (t->offset || t->byte_size) bad = "invalid tensor placement";
                spans[i].off = spans[i].end = 0;
                continue;
            }
            if (t->offset < h->data_offset || t->offset % QXF_ALIGN || !t->byte_size ||
                t->offset > h->file_size || t->byte_size > h->file_size - t->offset) { bad = "invalid tensor placement"; break; }
            uint64_t bv = 0, bb = 0;
            if (!qxf_type_block(t->flags, &bv, &bb) || t->dims[0] % bv || elems % bv ||
                (elems / bv) * bb != t->byte_size) { bad = "tensor byte size inconsistent with dimensions"; break; }
            spans[i].off = t->offset;
            spans[i].end = t->offset + t->byte_size;
        }
        if (!bad) {
            qsort(names, h->tensor_count, sizeof(*names), cmp_name);
            for (uint32_t i = 1; i < h->tensor_count; ++i)
                if (!strcmp(names[i - 1], names[i])) { bad = "duplicate tensor name"; break; }
        }
        if (!bad && !meta_only) {
            qsort(spans, h->tensor_count, sizeof(*spans), cmp_span);
            uint64_t prev = h->data_offset;
            for (uint32_t i = 0; i < h->tensor_count; ++i) {
                if (spans[i].off < prev) { bad = "overlapping tensor ranges"; break; }
                prev = spans[i].end;
            }
        }
        free(names);
        free(spans);
        if (bad) { set_err(err, err_len, bad); goto fail; }
    }
    out->map = (const uint8_t *)mmap(NULL, (size_t)h->file_size, PROT_READ, MAP_PRIVATE, out->fd, 0);
    if (out->map == MAP_FAILED) { out->map = NULL; set_err(err, err_len, "QXF file mapping failed"); goto fail; }
    return 1;
fail:
    qxf_close(out);
    return 0;
}

const qxf_dir_entry *qxf_find(const qxf_file *f, const char *name) {
    if (!f || !f->dir || !name) return NULL;
    for (uint32_t i = 0; i < f->header.tensor_count; ++i)
        if (!strcmp(f->dir[i].name, name)) return &f->dir[i];
    return NULL;
}

const uint8_t *qxf_data(const qxf_file *f, const qxf_dir_entry *t) {
    if (!f || !f->map || !t || !t->byte_size) return NULL;
    return f->map + t->offset;
}

int qxf_verify(const qxf_file *f, const qxf_dir_entry *t, char *err, uint64_t err_len) {
    const uint8_t *p = qxf_data(f, t);
    if (!p) { set_err(err, err_len, "invalid argument"); return 0; }
    if (qxf_fnv1a64(p, t->byte_size) != t->checksum) { set_err(err, err_len, "tensor checksum mismatch"); return 0; }
    return 1;
}
