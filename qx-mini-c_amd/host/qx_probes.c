/* Host side of the GPU path: QXF1 -> device upload, and the reference's probe
 * entry points (decode-block, final-head-probe, the full-MoE state loop) driving
 * the qxg C ABI.  JSON field names follow the reference's output so existing
 * consumers of those probes keep working. */
#include "qx_host.h"
#include "qxg.h"

#include <errno.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>

static void set_err(char *err, uint64_t n, const char *msg) {
    if (err && n) snprintf(err, (size_t)n, "%s", msg);
}

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

static int open_gpu(const char *path, int verify, qxg_ctx **ctx, qx_gpu_model_info *mi, char *err, uint64_t err_len) {
    if (!qxg_open(0, ctx, err, err_len)) return 0;
    if (!qx_gpu_load(*ctx, path, verify, mi, err, err_len)) { qxg_close(*ctx); *ctx = NULL; return 0; }
    return 1;
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

/* reference qx_read_exact_f32_sidecar (src/qx_format.c:5319-5344) */
static int read_sidecar(const char *path, float *v, uint32_t n, char *err, uint64_t err_len) {
    FILE *fp = fopen(path, "rb");
    if (!fp) { set_err(err, err_len, "cannot open F32 sidecar"); return 0; }
    struct stat st;
    if (fstat(fileno(fp), &st) != 0 || (uint64_t)st.st_size != (uint64_t)n * 4 || fread(v, 4, n, fp) != n) {
        fclose(fp); set_err(err, err_len, "F32 sidecar size or read mismatch"); return 0;
    }
    fclose(fp);
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) { set_err(err, err_len, "F32 sidecar contains non-finite value"); return 0; }
    return 1;
}

static int write_f32(const char *dir, const char *name, const float *v, uint32_t n, char *err, uint64_t err_len) {
    char p[1024];
    int len = snprintf(p, sizeof(p), "%s/%s.f32", dir, name);
    if (len < 0 || (size_t)len >= sizeof(p)) { set_err(err, err_len, "sidecar path too long"); return 0; }
    FILE *fp = fopen(p, "wb");
    if (!fp) { set_err(err, err_len, "cannot open sidecar for writing"); return 0; }
    int ok = fwrite(v, 4, n, fp) == n;
    if (fclose(fp) != 0) ok = 0;
    if (!ok) { remove(p); set_err(err, err_len, "cannot write sidecar"); }
    return ok;
}

static void remove_f32(const char *dir, const char *name) {
    char p[1024];
    snprintf(p, sizeof(p), "%s/%s.f32", dir, name);
    remove(p);
}

/* "f32" -> 0, "q8_k_compat" -> 1, anything else -> -1 (reference src/qx_format.c:5971-5973) */
static int activation_code(const char *s) {
    if (!s) return -1;
    return !strcmp(s, "f32") ? 0 : !strcmp(s, "q8_k_compat") ? 1 : -1;
}

int qx_dump_final_head_probe_summary(const char *path, const char *residual_path, const char *output_dir,
        const char *activation_mode, uint32_t top_n, FILE *out, char *err, uint64_t err_len) {
    const int act = activation_code(activation_mode);
    if (!path || !residual_path || !output_dir || !out || top_n == 0 || top_n > 32 || act < 0) {
        set_err(err, err_len, "invalid final head probe argument or activation mode"); return 0;
    }
    float res[2048], nrm[2048];
    if (!read_sidecar(residual_path, res, 2048, err, err_len)) return 0;
    qxg_ctx *ctx = NULL;
    qx_gpu_model_info mi;
    if (!open_gpu(path, 1, &ctx, &mi, err, err_len)) return 0;
    if (!mi.has_head) { qxg_close(ctx); set_err(err, err_len, "final head requires Q6_K output.weight"); return 0; }
    if (!qxg_set_activation(ctx, (uint32_t)act, err, err_len)) { qxg_close(ctx); return 0; }
    float *logits = (float *)malloc((size_t)mi.vocab * 4);
    uint32_t ids[32];
    double lg[32];
    int ok = logits && qxg_final_head(ctx, res, nrm, logits, top_n, ids, lg, err, err_len);
    qxg_close(ctx);
    if (ok && !write_f32(output_dir, "final-norm", nrm, 2048, err, err_len)) ok = 0;
    if (ok && !write_f32(output_dir, "logits", logits, mi.vocab, err, err_len)) { remove_f32(output_dir, "final-norm"); ok = 0; }
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

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int dump_vec(const char *dir, uint32_t step, uint32_t layer, const char *phase, const float *v, uint32_t n,
                    char *err, uint64_t err_len) {
    char name[128];
    snprintf(name, sizeof(name), "step-%u-layer-%u-%s", step, layer, phase);
    return write_f32(dir, name, v, n, err, err_len);
}

/* Full-MoE state loop on the GPU (reference src/qx_format.c:5970-6719 with
 * --full-moe [--final-head], INT8 KV, f32 or q8_k_compat activations, temperature 0). */
int qx_dump_prompt_state_loop_gpu(const char *path, const uint32_t *prompt, uint32_t n_prompt,
        uint32_t gen_steps, uint32_t ctx_tokens, const char *kv_format, const char *activation_format,
        int final_head, uint32_t top_n, const char *dump_dir, int bench, FILE *out, char *err, uint64_t err_len) {
    if (!path || !prompt || !out) { set_err(err, err_len, "invalid argument"); return 0; }
    if (!kv_format || strcmp(kv_format, "int8") != 0) { set_err(err, err_len, "the GPU state loop supports INT8 KV only"); return 0; }
    const int act = activation_code(activation_format);
    if (act < 0) { set_err(err, err_len, "unsupported activation format"); return 0; }
    if (gen_steps == 0 || n_prompt == 0) { set_err(err, err_len, "prompt state loop requires >= 1 prompt token and >= 1 generation step"); return 0; }
    if (ctx_tokens == 0 || ctx_tokens > 4096) { set_err(err, err_len, "state loop context must be between 1 and 4096"); return 0; }
    const uint32_t steps = n_prompt + gen_steps - 1;
    if (steps > ctx_tokens) { set_err(err, err_len, "steps exceed ctx"); return 0; }
    if (top_n == 0) top_n = 1;
    if (top_n > 32) top_n = 32;
    qxg_ctx *ctx = NULL;
    qx_gpu_model_info mi;
    double t_load = now_s();
    if (!open_gpu(path, 1, &ctx, &mi, err, err_len)) return 0;
    t_load = now_s() - t_load;
    if (!mi.has_embedding) { qxg_close(ctx); set_err(err, err_len, "token_embd.weight not found"); return 0; }
    if (!qxg_set_activation(ctx, (uint32_t)act, err, err_len)) { qxg_close(ctx); return 0; }
    if (final_head && !mi.has_head) { qxg_close(ctx); set_err(err, err_len, "final head requires Q6_K output.weight"); return 0; }
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= mi.vocab) { qxg_close(ctx); set_err(err, err_len, "prompt token out of range"); return 0; }
    if (!qxg_kv_create(ctx, mi.layers, ctx_tokens, 1, err, err_len)) { qxg_close(ctx); return 0; }
    float *x = (float *)malloc(2048 * 4), *a = (float *)malloc(2048 * 4), *y = (float *)malloc(2048 * 4);
    float *kqv = (float *)malloc(4096 * 4), *vcur = (float *)malloc(512 * 4), *moe = (float *)malloc(2048 * 4);
    float *logits = (float *)malloc((size_t)mi.vocab * 4);
    int ok = x && a && y && kqv && vcur && moe && logits;
    if (!ok) set_err(err, err_len, "out of memory");
    fprintf(out, "{\n  \"probe\": \"prompt_state_loop\",\n  \"backend\": \"hip-gfx950\",\n  \"layers\": %u,\n"
            "  \"ctx_tokens\": %u,\n  \"kv_format\": \"int8\",\n  \"activation_format\": \"%s\",\n  \"full_moe\": true,\n"
            "  \"final_head\": %s,\n  \"prompt_tokens\": %u,\n  \"generation_steps\": %u,\n  \"steps\": %u,\n  \"tokens\": [",
            mi.layers, ctx_tokens, act ? "q8_k_compat" : "f32", final_head ? "true" : "false", n_prompt, gen_steps, steps);
    uint32_t current = prompt[0];
    double t_loop = now_s();
    for (uint32_t s = 0; ok && s < steps; ++s) {
        if (s < n_prompt) current = prompt[s];
        const int sampling = s + 1 >= n_prompt;
        const int run_head = sampling && final_head;
        uint32_t ids[32];
        double lg[32];
        if (dump_dir && *dump_dir) {
            ok = qxg_embed_token(ctx, current, x, err, err_len);
            for (uint32_t l = 0; ok && l < mi.layers; ++l) {
                ok = dump_vec(dump_dir, s, l, "input", x, 2048, err, err_len) &&
                     qxg_attention_layer(ctx, l, s, x, a, kqv, vcur, err, err_len) &&
                     dump_vec(dump_dir, s, l, "v-cur", vcur, 512, err, err_len) &&
                     dump_vec(dump_dir, s, l, "kqv-out", kqv, 4096, err, err_len);
                if (!ok) break;
                for (int i = 0; i < 2048; ++i) x[i] += a[i];
                uint32_t eid[8];
                double ew[8];
                ok = dump_vec(dump_dir, s, l, "ffn-inp", x, 2048, err, err_len) &&
                     qxg_moe_layer(ctx, l, x, y, moe, eid, ew, err, err_len) &&
                     dump_vec(dump_dir, s, l, "ffn-moe-out", moe, 2048, err, err_len) &&
                     dump_vec(dump_dir, s, l, "output", y, 2048, err, err_len);
                memcpy(x, y, 2048 * 4);
            }
            if (ok && run_head) {
                ok = qxg_final_head(ctx, x, NULL, logits, top_n, ids, lg, err, err_len);
                char nm[64];
                snprintf(nm, sizeof(nm), "step-%u-logits", s);
                if (ok) ok = write_f32(dump_dir, nm, logits, mi.vocab, err, err_len);
            }
        } else {
            ok = qxg_decode_token(ctx, current, s, run_head, x, NULL, NULL, top_n, ids, lg, err, err_len);
        }
        if (!ok) break;
        fprintf(out, "%s{\"step\": %u, \"position\": %u, \"phase\": \"%s\", \"input_token\": %u", s ? ", " : "", s, s,
                sampling ? "generate" : "prefill", current);
        if (run_head) {
            fprintf(out, ", \"final_head\": {\"argmax_token\": %u, \"argmax_logit\": %.17g, \"top_tokens\": [", ids[0], lg[0]);
            for (uint32_t i = 0; i < top_n; ++i) fprintf(out, "%s{\"token\": %u, \"logit\": %.17g}", i ? ", " : "", ids[i], lg[i]);
            fprintf(out, "]}, \"selected_token\": %u}", ids[0]);
            current = ids[0];
        } else {
            fprintf(out, ", \"residual_checksum_after\": %llu, \"selected_token\": null}", (unsigned long long)qxf_fnv1a64(x, 2048 * 4));
        }
    }
    t_loop = now_s() - t_loop;
    if (ok) {
        fprintf(out, "],\n  \"final_token\": %u,\n  \"load_seconds\": %.6f,\n  \"loop_seconds\": %.6f", current, t_load, t_loop);
        if (bench && final_head) {
            uint32_t *gen = (uint32_t *)malloc((size_t)gen_steps * 4);
            float ms = 0.0f;
            if (gen && qxg_kv_create(ctx, mi.layers, ctx_tokens, 1, err, err_len) &&
                qxg_generate(ctx, prompt, n_prompt, gen_steps, 0, gen, &ms, err, err_len)) {
                fprintf(out, ",\n  \"bench\": {\"device_ms\": %.6f, \"steps\": %u, \"tokens_per_second\": %.3f, \"final_token\": %u}",
                        ms, steps, steps / (ms * 1e-3), gen[gen_steps - 1]);
            } else {
                ok = 0;
            }
            free(gen);
        }
        fprintf(out, "\n}\n");
    }
    free(x); free(a); free(y); free(kqv); free(vcur); free(moe); free(logits);
    qxg_close(ctx);
    return ok;
}

/* Q8_K blocks of the probe's fixed inputs, quantized on the GPU (reference
 * qx_dump_q8_k_activation_probe_summary, src/qx_format.c:4304-4345: same inputs,
 * injections, errors and JSON keys). */
int qx_dump_q8_k_activation_probe_gpu(uint32_t values, const char *inject, FILE *out, char *err, uint64_t err_len) {
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
        fprintf(out, "{\n  \"probe\": \"q8_k_activation\",\n  \"backend\": \"hip\",\n"
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
