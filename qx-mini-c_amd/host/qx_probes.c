/* Host side of the GPU path: QXF1 -> device upload, and the reference's probe entry
 * points decode-block, final-head-probe and q8-k-activation-probe driving the qxg C
 * ABI (the state loop and the stage probes have files of their own).  JSON field names
 * follow the reference's output so existing consumers of those probes keep working. */
#include "qx_util.h"

#include <errno.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>

#define set_err qxh_set_err

int qx_gpu_load(struct qxg_ctx *ctx, const char *path, int verify, qx_gpu_model_info *info, char *err, uint64_t err_len) {
    qxf_file f;
    if (!qxf_open(path, &f, err, err_len)) return 0;
    qx_gpu_model_info mi;
    memset(&mi, 0, sizeof(mi));
    int ok = 1;
    uint32_t max_layer_plus1 = 0;
    for (uint32_t i = 0; ok && i < f.header.tensor_count; ++i) {
        const qxf_dir_entry *t = &f.dir[i];
        if (verify && !qxf_verify(&f, t, err, err_len)) { ok = 0; break; }
        if (!qxg_upload_tensor(ctx, t->name, t->flags, t->dims, qxf_data(&f, t), t->byte_size, err, err_len)) { ok = 0; break; }
        mi.tensor_bytes += t->byte_size;
        ++mi.tensors;
        unsigned l;
        if (sscanf(t->name, "blk.%u.", &l) == 1 && l + 1 > max_layer_plus1) max_layer_plus1 = l + 1;
        if (!strcmp(t->name, "token_embd.weight")) mi.has_embedding = 1;
        if (!strcmp(t->name, "output.weight")) mi.has_head = 1;
    }
    if (ok) {
        mi.layers = max_layer_plus1;
        ok = qxg_bind_model(ctx, mi.layers, mi.has_embedding, mi.has_head, err, err_len);
    }
    if (ok) {
        mi.vocab = f.header.manifest.vocab;
        mi.experts = f.header.manifest.experts;
        if (info) *info = mi;
    }
    qxf_close(&f);
    return ok;
}


int qx_dump_decode_block_summary(const char *path, const char *name, uint64_t block_index, FILE *out, char *err, uint64_t err_len) {
    qxf_file f;
    if (!path || !name || !out) { set_err(err, err_len, "invalid argument"); return 0; }
    if (!qxf_open(path, &f, err, err_len)) return 0;
    const qxf_dir_entry *t = qxf_find(&f, name);
    uint64_t bv = 0, bb = 0;
    if (!t) { qxf_close(&f); set_err(err, err_len, "tensor not found"); return 0; }
    if (!qxf_type_block(t->flags, &bv, &bb) || bv != 256 ||
        (t->flags != QXT_Q4_K && t->flags != QXT_Q6_K && t->flags != QXT_IQ2_XS && t->flags != QXT_IQ3_XXS && t->flags != QXT_IQ4_XS)) {
        qxf_close(&f); set_err(err, err_len, "unsupported GGML type for decode-block"); return 0;
    }
    if (block_index >= t->byte_size / bb) { qxf_close(&f); set_err(err, err_len, "block out of range"); return 0; }
    qxg_ctx *ctx = NULL;
    if (!qxg_open(0, &ctx, err, err_len)) { qxf_close(&f); return 0; }
    const uint8_t *raw = qxf_data(&f, t) + block_index * bb;
    float v[256];
    int ok = qxg_dequant_blocks(ctx, t->flags, raw, 1, v, err, err_len);
    qxg_close(ctx);
    if (ok) {
        double sum = 0.0;
        float mn = v[0], mx = v[0];
        for (int i = 0; i < 256; ++i) { sum += v[i]; if (v[i] < mn) mn = v[i]; if (v[i] > mx) mx = v[i]; }
        fprintf(out, "{\n  \"tensor\": \"%s\",\n  \"ggml_type\": %u,\n  \"decoded\": true,\n  \"backend\": \"hip\",\n", t->name, t->flags);
        fprintf(out, "  \"block_index\": %llu,\n  \"block_offset\": %llu,\n  \"block_byte_size\": %llu,\n  \"values\": 256,\n",
                (unsigned long long)block_index, (unsigned long long)(t->offset + block_index * bb), (unsigned long long)bb);
        fprintf(out, "  \"sum\": %.9g,\n  \"min\": %.9g,\n  \"max\": %.9g,\n", sum, (double)mn, (double)mx);
        fprintf(out, "  \"raw_checksum\": %llu,\n  \"f32_checksum\": %llu,\n  \"first8\": [",
                (unsigned long long)qxf_fnv1a64(raw, bb), (unsigned long long)qxf_fnv1a64(v, sizeof(v)));
        for (int i = 0; i < 8; ++i) fprintf(out, "%s%.9g", i ? ", " : "", (double)v[i]);
        fprintf(out, "]\n}\n");
    }
    qxf_close(&f);
    return ok;
}

int qx_dump_final_head_probe_summary(const char *path, const char *residual_path, const char *output_dir,
        const char *activation_mode, uint32_t top_n, FILE *out, char *err, uint64_t err_len) {
    const int act = qxh_activation_code(activation_mode);
    if (!path || !residual_path || !output_dir || !out || top_n == 0 || top_n > 32 || act < 0) {
        set_err(err, err_len, "invalid final head probe argument or activation mode"); return 0;
    }
    float res[2048], nrm[2048];
    if (!qxh_read_sidecar(residual_path, res, 2048, err, err_len)) return 0;
    qxg_ctx *ctx = NULL;
    qx_gpu_model_info mi;
    if (!qxh_open_gpu(path, 1, &ctx, &mi, err, err_len)) return 0;
    if (!mi.has_head) { qxg_close(ctx); set_err(err, err_len, "final head requires Q6_K output.weight"); return 0; }
    if (!qxg_set_activation(ctx, (uint32_t)act, err, err_len)) { qxg_close(ctx); return 0; }
    float *logits = (float *)malloc((size_t)mi.vocab * 4);
    uint32_t ids[32];
    double lg[32];
    int ok = logits && qxg_final_head(ctx, res, nrm, logits, top_n, ids, lg, err, err_len);
    qxg_close(ctx);
    if (ok && !qxh_write_f32(output_dir, "final-norm", nrm, 2048, err, err_len)) ok = 0;
    if (ok && !qxh_write_f32(output_dir, "logits", logits, mi.vocab, err, err_len)) { qxh_remove_f32(output_dir, "final-norm"); ok = 0; }
    if (ok) {
        double ss = 0.0, ns = 0.0;
        for (int i = 0; i < 2048; ++i) { ss += (double)res[i] * res[i]; ns += (double)nrm[i] * nrm[i]; }
        fprintf(out, "{\"probe\":\"final_head\",\"backend\":\"hip\",\"input_dims\":2048,\"vocab_size\":%u,"
                "\"activation_mode\":\"%s\",\"lm_head_kernel\":\"%s\",\"input_rms\":%.17g,"
                "\"normalized_l2\":%.17g,\"residual_checksum\":%llu,\"normalized_checksum\":%llu,"
                "\"logits_checksum\":%llu,\"argmax_token\":%u,\"argmax_logit\":%.17g,\"top_tokens\":[",
                mi.vocab, act ? "q8_k_compat" : "f32", act ? "q6_k_q8_k_hip_dot4" : "q6_k_hip_dot4",
                sqrt(ss / 2048.0 + 1.0e-6), sqrt(ns), (unsigned long long)qxf_fnv1a64(res, sizeof(res)),
                (unsigned long long)qxf_fnv1a64(nrm, sizeof(nrm)), (unsigned long long)qxf_fnv1a64(logits, (uint64_t)mi.vocab * 4),
                ids[0], lg[0]);
        for (uint32_t i = 0; i < top_n; ++i) fprintf(out, "%s{\"token\":%u,\"logit\":%.17g}", i ? "," : "", ids[i], lg[i]);
        fprintf(out, "]}\n");
    }
    free(logits);
    return ok;
}

/* Q8_K blocks of the probe's fixed inputs, quantized on the GPU (reference
 * qx_dump_q8_k_activation_probe_summary, src/qx_format.c:4304-4345: same inputs,
 * injections, errors and JSON keys). */
int qx_dump_q8_k_activation_probe_summary(uint32_t values, const char *inject, FILE *out, char *err, uint64_t err_len) {
    static const char *const kinds[] = {"none", "zero", "nan", "inf", "positive", "negative", "edge"};
    int kind = -1;
    for (int i = 0; inject && i < 7; ++i) if (!strcmp(inject, kinds[i])) kind = i;
    if (!out || !inject || values == 0) { set_err(err, err_len, "invalid Q8_K activation probe size"); return 0; }
    if (values > 4096) { set_err(err, err_len, "Q8_K activation workspace is too small"); return 0; }
    if (kind < 0) { set_err(err, err_len, "invalid Q8_K activation injection"); return 0; }
    float x[4096];
    for (uint32_t i = 0; i < values; ++i) {
        switch (kind) {
        case 1: x[i] = 0.0f; break;
        case 4: x[i] = (float)(i % 127u) / 127.0f; break;
        case 5: x[i] = -(float)(i % 127u) / 127.0f; break;
        case 6: x[i] = i % 2u ? 1.0f : -1.0f; break;
        default: x[i] = (float)((int32_t)(i % 251u) - 125) / 127.0f; break;
        }
    }
    if (kind == 2) x[values / 2] = NAN;
    if (kind == 3) x[values / 2] = INFINITY;
    qxg_ctx *ctx = NULL;
    if (!qxg_open(0, &ctx, err, err_len)) return 0;
    const uint32_t blocks = values / 256;
    uint8_t *b = (uint8_t *)malloc((size_t)(blocks ? blocks : 1) * 292);
    int ok = b && qxg_q8k_quantize(ctx, x, values, b, err, err_len);
    qxg_close(ctx);
    if (ok) {
        int64_t qsum = 0;
        for (uint32_t k = 0; k < blocks; ++k)
            for (int i = 0; i < 256; ++i) qsum += (int8_t)b[292ull * k + 4 + i];
        float d0;
        memcpy(&d0, b, 4);
        fprintf(out, "{\n  \"probe\": \"q8_k_activation\",\n"
                "  \"activation_format\": \"q8_k_compat\",\n  \"values\": %u,\n  \"blocks\": %u,\n"
                "  \"block_bytes\": 292,\n  \"workspace_bytes\": %u,\n  \"first_scale\": %.9g,\n"
                "  \"quant_sum\": %lld,\n  \"finite\": true,\n  \"block_hex\": \"",
                values, blocks, blocks * 292u, d0, (long long)qsum);
        for (uint32_t i = 0; i < blocks * 292u; ++i) fprintf(out, "%02x", b[i]);
        fprintf(out, "\",\n  \"checksum\": %llu\n}\n", (unsigned long long)qxf_fnv1a64(b, (uint64_t)blocks * 292));
    }
    free(b);
    return ok;
}
