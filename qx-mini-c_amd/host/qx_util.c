/* Helpers shared by the host probe files. */
#include "qx_util.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>

void qxh_set_err(char *err, uint64_t n, const char *msg) {
    if (err && n) snprintf(err, (size_t)n, "%s", msg);
}

int qxh_read_sidecar(const char *path, float *v, uint32_t n, char *err, uint64_t err_len) {
    if (!path || !*path || !v || n == 0) { qxh_set_err(err, err_len, "invalid F32 sidecar argument"); return 0; }
    FILE *fp = fopen(path, "rb");
    if (!fp) { qxh_set_err(err, err_len, "cannot open F32 sidecar"); return 0; }
    struct stat st;
    if (fstat(fileno(fp), &st) != 0 || (uint64_t)st.st_size != (uint64_t)n * 4 || fread(v, 4, n, fp) != n) {
        fclose(fp); qxh_set_err(err, err_len, "F32 sidecar size or read mismatch"); return 0;
    }
    fclose(fp);
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) { qxh_set_err(err, err_len, "F32 sidecar contains non-finite value"); return 0; }
    return 1;
}

int qxh_write_f32(const char *dir, const char *name, const float *v, uint64_t n, char *err, uint64_t err_len) {
    char p[1024];
    int len = snprintf(p, sizeof(p), "%s/%s.f32", dir, name);
    if (len < 0 || (size_t)len >= sizeof(p)) { qxh_set_err(err, err_len, "sidecar path too long"); return 0; }
    FILE *fp = fopen(p, "wb");
    if (!fp) { qxh_set_err(err, err_len, "cannot open sidecar for writing"); return 0; }
    int ok = fwrite(v, 4, (size_t)n, fp) == (size_t)n;
    if (fclose(fp) != 0) ok = 0;
    if (!ok) { remove(p); qxh_set_err(err, err_len, "cannot write sidecar"); }
    return ok;
}

void qxh_remove_f32(const char *dir, const char *name) {
    char p[1024];
    snprintf(p, sizeof(p), "%s/%s.f32", dir, name);
    remove(p);
}

int qxh_activation_code(const char *s) {
    if (!s) return -1;
    return !strcmp(s, "f32") ? 0 : !strcmp(s, "q8_k_compat") ? 1 : -1;
}

int qxh_open_gpu(const char *path, int verify, qxg_ctx **ctx, qx_gpu_model_info *mi, char *err, uint64_t err_len) {
    if (!qxg_open(0, ctx, err, err_len)) return 0;
    if (!qx_gpu_load(*ctx, path, verify, mi, err, err_len)) { qxg_close(*ctx); *ctx = NULL; return 0; }
    return 1;
}

double qxh_now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

uint32_t qxh_projection_family_bit(uint32_t t) {
    return t == QXT_IQ4_XS ? 1u : t == QXT_Q5_K ? 2u : t == QXT_Q6_K ? 4u : 0u;
}

const char *qxh_projection_kernel_label(uint32_t mask, int f32_used) {
    static const char *const plain[8] = {"not_used", "iq4_xs_q8_k", "q5_k_q8_k", "iq4_xs_q5_k_q8_k", "q6_k_q8_k",
                                         "iq4_xs_q6_k_q8_k", "q5_k_q6_k_q8_k", "iq4_xs_q5_k_q6_k_q8_k"};
    static const char *const mixed[8] = {"dequant_f32", "iq4_xs_q8_k_with_f32_fallback", "q5_k_q8_k_with_f32_fallback",
                                         "iq4_xs_q5_k_q8_k_with_f32_fallback", "q6_k_q8_k_with_f32_fallback",
                                         "iq4_xs_q6_k_q8_k_with_f32_fallback", "q5_k_q6_k_q8_k_with_f32_fallback",
                                         "iq4_xs_q5_k_q6_k_q8_k_with_f32_fallback"};
    if (mask > 7u) return "invalid_projection_kernel_state";
    return f32_used ? mixed[mask] : plain[mask];
}

const char *qxh_projection_tensor_kernel_label(uint32_t t, int use_q8_k) {
    if (!use_q8_k) return "dequant_f32";
    const uint32_t fam = qxh_projection_family_bit(t);
    return fam ? qxh_projection_kernel_label(fam, 0) : "dequant_f32";
}

const qxf_dir_entry *qxh_layer_tensor(const qxf_file *f, uint32_t layer, const char *suffix) {
    char name[QXF_NAME_MAX];
    snprintf(name, sizeof(name), "blk.%u.%s", layer, suffix);
    return qxf_find(f, name);
}

void qxh_json_string(FILE *out, const char *s) {
    fputc('"', out);
    for (const unsigned char *p = (const unsigned char *)s; p && *p; ++p) {
        switch (*p) {
        case '"': fputs("\\\"", out); break;
        case '\\': fputs("\\\\", out); break;
        case '\n': fputs("\\n", out); break;
        case '\r': fputs("\\r", out); break;
        case '\t': fputs("\\t", out); break;
        default:
            if (*p < 0x20) fprintf(out, "\\u%04x", *p);
            else fputc(*p, out);
        }
    }
    fputc('"', out);
}
