/* The reference's attention-stage and MoE-stage probes (include/qx_format.h:160-161 of
 * the reference) on the GPU: same arguments, validation messages, sidecar files and
 * JSON keys; the stage arithmetic runs in qxg_attention_stage / qxg_moe_stage. */
#include "qx_util.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* reference qx_dump_attention_stage_probe_summary (src/qx_format.c:5478-5586) */
int qx_dump_attention_stage_probe_summary(const char *path, uint32_t layer, const char *layer_input_path,
        const char *output_dir, const char *activation_mode, const char *kv_format, FILE *out, char *err,
        uint64_t err_len) {
    const int use_q8 = activation_mode && !strcmp(activation_mode, "q8_k_compat");
    const int use_f16 = kv_format && !strcmp(kv_format, "f16");
    if (!path || !layer_input_path || !output_dir || !out ||
        (!use_q8 && (!activation_mode || strcmp(activation_mode, "f32") != 0)) ||
        (!use_f16 && (!kv_format || strcmp(kv_format, "f32") != 0))) {
        qxh_set_err(err, err_len, "invalid attention stage probe argument, activation mode, or KV format");
        return 0;
    }
    qxf_file f;
    if (!qxf_open(path, &f, err, err_len)) return 0;
    const qxf_manifest *m = &f.header.manifest;
    const uint32_t hidden = m->hidden, qh = m->q_heads, kvh = m->kv_heads, hd = m->head_dim;
    if (layer >= m->layers || hidden == 0 || hidden > 2048 || qh == 0 || kvh == 0 || hd == 0 || qh % kvh != 0 ||
        qh > UINT32_MAX / hd || kvh > UINT32_MAX / hd) {
        qxf_close(&f); qxh_set_err(err, err_len, "invalid attention stage layer or dimensions"); return 0;
    }
    const uint32_t q_values = qh * hd, kv_values = kvh * hd;
    /* the device kernels are built for the Qwen3-30B-A3B attention geometry */
    if (hidden != 2048 || qh != 32 || kvh != 4 || hd != 128) {
        qxf_close(&f); qxh_set_err(err, err_len, "unsupported attention stage dimensions"); return 0;
    }
    const qxf_dir_entry *nt = qxh_layer_tensor(&f, layer, "attn_norm.weight");
    const qxf_dir_entry *vt = qxh_layer_tensor(&f, layer, "attn_v.weight");
    const qxf_dir_entry *ot = qxh_layer_tensor(&f, layer, "attn_output.weight");
    if (!nt || !vt || !ot || vt->dims[0] != hidden || vt->dims[1] != kv_values || ot->dims[0] != q_values ||
        ot->dims[1] != hidden) {
        qxf_close(&f); qxh_set_err(err, err_len, "unsupported attention stage tensor layout"); return 0;
    }
    const uint32_t vtype = vt->flags, otype = ot->flags;
    qxf_close(&f);
    float x[2048], norm[2048], vcur[512], kqv[4096], attn[2048], ffn[2048];
    if (!qxh_read_sidecar(layer_input_path, x, hidden, err, err_len)) return 0;
    qxg_ctx *ctx = NULL;
    qx_gpu_model_info mi;
    if (!qxh_open_gpu(path, 1, &ctx, &mi, err, err_len)) return 0;
    int ok = qxg_set_activation(ctx, (uint32_t)use_q8, err, err_len) &&
             qxg_attention_stage(ctx, layer, use_f16, x, norm, vcur, kqv, attn, ffn, err, err_len);
    qxg_close(ctx);
    if (!ok) return 0;
    char name[64];
    static const char *const names[5] = {"attn_norm", "Vcur", "kqv_out", "attn_out", "ffn_inp"};
    const float *vecs[5] = {norm, vcur, kqv, attn, ffn};
    const uint32_t counts[5] = {hidden, kv_values, q_values, hidden, hidden};
    for (int i = 0; i < 5; ++i) {
        snprintf(name, sizeof(name), "%s-%u", names[i], layer);
        if (!qxh_write_f32(output_dir, name, vecs[i], counts[i], err, err_len)) return 0;
    }
    /* the input's RMS as qx_apply_f32_rmsnorm reports it (src/qx_format.c:3363-3365); the
     * probes are the projections' row sums (src/qx_format.c:4276-4287, here of the f32 rows) */
    double ss = 0.0, vprobe = 0.0, oprobe = 0.0;
    for (uint32_t i = 0; i < hidden; ++i) ss += (double)x[i] * (double)x[i];
    for (uint32_t i = 0; i < kv_values; ++i) vprobe += (double)vcur[i];
    for (uint32_t i = 0; i < hidden; ++i) oprobe += (double)attn[i];
    const uint32_t fam = qxh_projection_family_bit(vtype) | qxh_projection_family_bit(otype);
    const int f32_used = use_q8 && (!qxh_projection_family_bit(vtype) || !qxh_projection_family_bit(otype));
    fprintf(out, "{\"probe\":\"attention_stage\",\"layer\":%u,\"hidden\":%u,\"q_values\":%u,\"kv_values\":%u,"
            "\"activation_mode\":\"%s\",\"kv_format\":\"%s\",\"projection_kernel\":\"%s\",\"v_projection_kernel\":\"%s\","
            "\"output_projection_kernel\":\"%s\",\"single_token_softmax\":1.0,\"norm_rms\":%.9g,"
            "\"v_probe\":%.9g,\"output_probe\":%.9g,\"v_count\":%u,\"output_count\":%u}\n",
            layer, hidden, q_values, kv_values, activation_mode, kv_format,
            use_q8 ? qxh_projection_kernel_label(fam, f32_used) : "dequant_f32",
            qxh_projection_tensor_kernel_label(vtype, use_q8), qxh_projection_tensor_kernel_label(otype, use_q8),
            sqrt(ss / (double)hidden + 1.0e-6), vprobe, oprobe, kv_values, hidden);
    return 1;
}

/* reference qx_dump_moe_stage_probe_summary (src/qx_format.c:5588-5725) */
int qx_dump_moe_stage_probe_summary(const char *path, uint32_t layer, const char *ffn_input_path,
        const char *output_dir, const char *activation_mode, FILE *out, char *err, uint64_t err_len) {
    const int use_q8 = activation_mode && !strcmp(activation_mode, "q8_k_compat");
    if (!path || !ffn_input_path || !output_dir || !out ||
        (!use_q8 && (!activation_mode || strcmp(activation_mode, "f32") != 0))) {
        qxh_set_err(err, err_len, "invalid MoE stage probe argument or activation mode"); return 0;
    }
    qxf_file f;
    if (!qxf_open(path, &f, err, err_len)) return 0;
    const uint32_t hidden = f.header.manifest.hidden;
    if (hidden == 0 || layer >= f.header.manifest.layers) {
        qxf_close(&f); qxh_set_err(err, err_len, "invalid MoE stage layer"); return 0;
    }
    const qxf_dir_entry *nt = qxh_layer_tensor(&f, layer, "ffn_norm.weight");
    const qxf_dir_entry *rt = qxh_layer_tensor(&f, layer, "ffn_gate_inp.weight");
    const qxf_dir_entry *gt = qxh_layer_tensor(&f, layer, "ffn_gate_exps.weight");
    const qxf_dir_entry *ut = qxh_layer_tensor(&f, layer, "ffn_up_exps.weight");
    const qxf_dir_entry *dt = qxh_layer_tensor(&f, layer, "ffn_down_exps.weight");
    const uint32_t E = rt && rt->rank > 1 ? (uint32_t)rt->dims[1] : 0u;
    const uint32_t F = gt && gt->rank > 1 ? (uint32_t)gt->dims[1] : 0u;
    if (!nt || !rt || !gt || !ut || !dt || E < 8 || E > 128 || F == 0 || rt->flags != 0 || rt->dims[0] != hidden ||
        rt->byte_size != (uint64_t)hidden * E * 4 || gt->rank < 3 || ut->rank < 3 || dt->rank < 3 ||
        gt->dims[0] != hidden || gt->dims[1] != F || gt->dims[2] != E || ut->dims[0] != hidden || ut->dims[1] != F ||
        ut->dims[2] != E || dt->dims[0] != F || dt->dims[1] != hidden || dt->dims[2] != E) {
        qxf_close(&f); qxh_set_err(err, err_len, "unsupported MoE stage tensor layout"); return 0;
    }
    const uint32_t tg = gt->flags, tu = ut->flags, td = dt->flags;
    qxf_close(&f);
    if (hidden != 2048 || F != 768) { qxh_set_err(err, err_len, "unsupported MoE stage tensor layout"); return 0; }
    float x[2048];
    if (!qxh_read_sidecar(ffn_input_path, x, hidden, err, err_len)) return 0;
    float *blk = (float *)malloc((size_t)QXG_MOE_STAGE_FLOATS(E) * 4);
    if (!blk) { qxh_set_err(err, err_len, "out of memory"); return 0; }
    qxg_ctx *ctx = NULL;
    qx_gpu_model_info mi;
    uint32_t ids[8];
    int ok = qxh_open_gpu(path, 1, &ctx, &mi, err, err_len);
    if (ok) {
        ok = qxg_set_activation(ctx, (uint32_t)use_q8, err, err_len) && qxg_moe_stage(ctx, layer, x, blk, ids, err, err_len);
        qxg_close(ctx);
    }
    static const char *const names[12] = {"ffn_norm", "ffn_moe_logits", "ffn_moe_probs", "ffn_moe_topk",
                                          "ffn_moe_weights", "ffn_moe_weights_sum", "ffn_moe_weights_norm",
                                          "ffn_moe_gate", "ffn_moe_up", "ffn_moe_swiglu", "ffn_moe_down",
                                          "ffn_moe_weighted"};
    const uint64_t counts[12] = {hidden, E, E, 8, 8, 1, 8, 8ull * F, 8ull * F, 8ull * F, 8ull * hidden, 8ull * hidden};
    uint32_t written = 0;
    const float *p = blk, *wnorm = NULL;
    char name[64];
    for (int i = 0; ok && i < 12; ++i) {
        if (i == 6) wnorm = p;
        snprintf(name, sizeof(name), "%s-%u", names[i], layer);
        ok = qxh_write_f32(output_dir, name, p, counts[i], err, err_len);
        written += ok ? 1u : 0u;
        p += counts[i];
    }
    if (ok) {
        const int gu_q8 = use_q8 && ((tg == QXT_IQ2_XS && tu == QXT_IQ2_XS) || (tg == QXT_IQ2_S && tu == QXT_IQ2_S));
        const int dn_q8 = use_q8 && (td == QXT_IQ3_XXS || td == QXT_IQ3_S || td == QXT_IQ4_XS);
        const int q8_used = gu_q8 || dn_q8, f32_used = !gu_q8 || !dn_q8;
        /* kernel labels (src/qx_format.c:5685-5717) */
        const char *label = "dequant_f32";
        if (q8_used && f32_used) label = "q8_k_expert_kernels_with_f32_fallback";
        else if (q8_used && tg == QXT_IQ2_XS && td == QXT_IQ3_XXS) label = "iq2_xs_q8_k_and_iq3_xxs_q8_k";
        else if (q8_used && tg == QXT_IQ2_S && td == QXT_IQ4_XS) label = "iq2_s_q8_k_and_iq4_xs_q8_k";
        else if (q8_used && tg == QXT_IQ2_XS && td == QXT_IQ3_S) label = "iq2_xs_q8_k_and_iq3_s_q8_k";
        else if (q8_used && tg == QXT_IQ2_S && td == QXT_IQ3_S) label = "iq2_s_q8_k_and_iq3_s_q8_k";
        else if (q8_used) label = "q8_k_expert_kernels";
        fprintf(out, "{\"probe\":\"moe_stage\",\"layer\":%u,\"input_count\":%u,\"experts\":%u,\"experts_used\":8,"
                "\"intermediate\":%u,\"activation_mode\":\"%s\",\"projection_kernel\":\"%s\","
                "\"gate_up_projection_kernel\":\"%s\",\"down_projection_kernel\":\"%s\",\"gate_ggml_type\":%u,"
                "\"up_ggml_type\":%u,\"down_ggml_type\":%u,\"selected_experts\":[",
                layer, hidden, E, F, activation_mode, label,
                gu_q8 ? (tg == QXT_IQ2_XS ? "iq2_xs_q8_k" : "iq2_s_q8_k") : "dequant_f32",
                dn_q8 ? (td == QXT_IQ3_XXS ? "iq3_xxs_q8_k" : td == QXT_IQ3_S ? "iq3_s_q8_k" : "iq4_xs_q8_k") : "dequant_f32",
                tg, tu, td);
        for (int r = 0; r < 8; ++r) fprintf(out, "%s%u", r ? "," : "", ids[r]);
        fprintf(out, "],\"routing_weights\":[");
        for (int r = 0; r < 8; ++r) fprintf(out, "%s%.9g", r ? "," : "", (double)wnorm[r]);
        fprintf(out, "],\"sidecars_written\":%u}\n", written);
    }
    free(blk);
    return ok;
}
