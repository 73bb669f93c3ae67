/* The reference's state-loop probes (include/qx_format.h:157-158 of the reference) on
 * the GPU: qx_dump_prompt_state_loop_probe_summary and its one-token wrapper
 * qx_dump_state_loop_probe_summary, with the reference's prototypes, validation
 * messages, JSON keys, residual dumps, KV snapshots (QXKVSNP1) and residual replay.
 *
 * With --final-head on the persistent path (the benchmark mix in f32) the whole loop is one
 * launch of the persistent decode, its argmax feeding each next token on the device, that
 * records every step's per-layer entries (qxg_generate_recorded): the layer outputs, the
 * attention and MoE halves, the routing, the heads' softmax sums, the head's norm, logits and
 * top tokens; the K/V rows are read back per layer after it.  Otherwise each step is one
 * qxg_decode_token call followed by the same readbacks for that step.  --bench times the
 * device work (the launch, or the per-step calls with their readbacks; the phases from the
 * device clock at each step's start in the one-launch mode) and reports the loop's wall time,
 * JSON formatting included, apart.  Residual
 * replay (--start-layer / --residual-in) and --dump-residuals, which need stage vectors the
 * fused step does not keep (v-cur, kqv-out), run through the per-layer seams
 * (qxg_attention_layer_ex, qxg_moe_layer, qxg_final_head).  The GPU path implements
 * --full-moe with INT8 KV; the reference's probe-level skeleton modes (without --full-moe)
 * are rejected with an error. */
#include "qx_util.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define NAME_MAX_LEN 96
#define FNV_OFFSET 1469598103934665603ull
#define FNV_PRIME 1099511628211ull

/* reference qx_deterministic_input (src/qx_format.c:2267-2271): a 32-bit LCG step, its
 * high half mapped to [-1, 1) */
static float det_input(uint32_t *st) {
    *st = *st * 1664525u + 1013904223u;
    return (float)((int)((*st >> 16) & 0xffffu) - 32768) / 32768.0f;
}

typedef struct { uint32_t token; double logit; uint64_t checksum; } top_token;

/* The scan that picks the next token when the state loop runs without --final-head
 * (qx_collect_top_logits / qx_logit_row_score, src/qx_format.c:2936-3006): rows
 * 0 .. scan-1 of the head tensor (output.weight, else lm_head.weight, else the tied
 * token_embd.weight), each scored by its first (at most 4) decoded blocks against the
 * LCG inputs seeded with seed ^ token, times the residual probe.  The blocks are decoded
 * on the device once per run (qxg_dequant_blocks); the scores per step on the host. */
typedef struct {
    const qxf_dir_entry *lm;
    uint32_t scan, blocks;
    float *vals;              /* [scan][blocks * 256] */
    uint64_t *row_fnv;        /* [scan] */
} probe_scan;

static int probe_scan_init(qxg_ctx *ctx, const qxf_file *f, uint32_t scan, probe_scan *ps, char *err, uint64_t n) {
    memset(ps, 0, sizeof(*ps));
    const qxf_dir_entry *lm = qxf_find(f, "output.weight");
    if (!lm) lm = qxf_find(f, "lm_head.weight");
    if (!lm) lm = qxf_find(f, "token_embd.weight");
    if (!lm) { qxh_set_err(err, n, "lm head/output/token embedding tensor not found"); return 0; }
    const uint32_t vocab = f->header.manifest.vocab ? f->header.manifest.vocab : (uint32_t)lm->dims[1];
    if (scan == 0) scan = 64;
    if (scan > vocab) scan = vocab;
    uint64_t bv = 0, bb = 0;
    if (!qxf_type_block(lm->flags, &bv, &bb) || bv != 256 || (lm->flags != QXT_Q6_K && lm->flags != QXT_Q4_K)) {
        qxh_set_err(err, n, "unsupported head tensor for the token scan"); return 0;
    }
    const uint64_t row = lm->byte_size / vocab, per_row = row / bb;
    ps->lm = lm;
    ps->scan = scan;
    ps->blocks = (uint32_t)(per_row < 4 ? per_row : 4);
    ps->vals = (float *)malloc((size_t)scan * ps->blocks * 256 * 4);
    ps->row_fnv = (uint64_t *)malloc((size_t)scan * 8);
    uint8_t *raw = (uint8_t *)malloc((size_t)scan * ps->blocks * bb);
    if (!ps->vals || !ps->row_fnv || !raw) { free(raw); qxh_set_err(err, n, "out of memory"); return 0; }
    const uint8_t *base = qxf_data(f, lm);
    for (uint32_t t = 0; t < scan; ++t) {
        memcpy(raw + (uint64_t)t * ps->blocks * bb, base + (uint64_t)t * row, (size_t)(ps->blocks * bb));
        ps->row_fnv[t] = qxf_fnv1a64(base + (uint64_t)t * row, row);
    }
    const int ok = qxg_dequant_blocks(ctx, lm->flags, raw, (uint64_t)scan * ps->blocks, ps->vals, err, n);
    free(raw);
    return ok;
}

static void probe_scan_free(probe_scan *ps) {
    free(ps->vals);
    free(ps->row_fnv);
}

/* top_n (<= scan) best rows by score, ties keeping the earlier row */
static uint32_t probe_scan_top(const probe_scan *ps, double activation, uint32_t top_n, uint32_t seed, top_token *top) {
    if (top_n == 0) top_n = 1;
    if (top_n > ps->scan) top_n = ps->scan;
    for (uint32_t i = 0; i < top_n; ++i) { top[i].token = 0; top[i].logit = -1.0e300; top[i].checksum = 0; }
    for (uint32_t t = 0; t < ps->scan; ++t) {
        uint32_t st = (seed ? seed : 1u) ^ t;
        double score = 0.0;
        const float *v = ps->vals + (uint64_t)t * ps->blocks * 256;
        for (uint32_t i = 0; i < ps->blocks * 256; ++i) score += (double)v[i] * (double)det_input(&st);
        const double logit = score * activation;
        for (uint32_t i = 0; i < top_n; ++i) {
            if (logit > top[i].logit) {
                for (uint32_t j = top_n - 1; j > i; --j) top[j] = top[j - 1];
                top[i].token = t; top[i].logit = logit; top[i].checksum = ps->row_fnv[t];
                break;
            }
        }
    }
    return top_n;
}

/* reference qx_sample_from_top (src/qx_format.c:3045-3084): argmax at temperature <= 0,
 * else one LCG draw against the tempered softmax of the candidates */
static uint32_t sample_from_top(const top_token *top, uint32_t k, double temperature, uint32_t seed) {
    if (k == 0) k = 1;
    if (temperature <= 0.0) return top[0].token;
    double mx = top[0].logit, p[32], sum = 0.0;
    for (uint32_t i = 1; i < k; ++i) if (top[i].logit > mx) mx = top[i].logit;
    for (uint32_t i = 0; i < k; ++i) { p[i] = exp((top[i].logit - mx) / temperature); sum += p[i]; }
    if (sum <= 0.0) sum = 1.0;
    for (uint32_t i = 0; i < k; ++i) p[i] /= sum;
    uint32_t st = seed ? seed : 1u;
    const double u = ((double)det_input(&st) + 1.0) * 0.5;
    double acc = 0.0;
    uint32_t rank = k - 1;
    for (uint32_t i = 0; i < k; ++i) {
        acc += p[i];
        if (u <= acc) { rank = i; break; }
    }
    return top[rank].token;
}

/* token piece from a "id<TAB>piece" sidecar with \t \n \r \\ escapes
 * (qx_lookup_token_piece_sidecar, src/qx_format.c:3138-3181), else "<tok_ID>" */
static const char *token_piece(const char *tokens_path, uint32_t id, char *buf, size_t cap, const char **source) {
    *source = "fallback_token_id";
    FILE *fp = tokens_path ? fopen(tokens_path, "rb") : NULL;
    if (fp) {
        char line[8192];
        while (fgets(line, sizeof(line), fp)) {
            if (line[0] == '#') continue;
            char *tab = strchr(line, '\t');
            if (!tab) continue;
            *tab = 0;
            if ((uint32_t)strtoul(line, NULL, 10) != id) continue;
            char *val = tab + 1;
            size_t n = strlen(val);
            while (n && (val[n - 1] == '\n' || val[n - 1] == '\r')) val[--n] = 0;
            size_t w = 0;
            for (size_t r = 0; val[r] && w + 1 < cap; ++r) {
                char ch = val[r];
                if (ch == '\\' && val[r + 1]) {
                    ++r;
                    ch = val[r] == 't' ? '\t' : val[r] == 'n' ? '\n' : val[r] == 'r' ? '\r' : val[r];
                }
                buf[w++] = ch;
            }
            buf[w] = 0;
            fclose(fp);
            *source = "sidecar";
            return buf;
        }
        fclose(fp);
    }
    snprintf(buf, cap, "<tok_%u>", id);
    return buf;
}

static int dump_vec(const char *dir, uint32_t step, uint32_t layer, const char *phase, const float *v, uint32_t n,
                    char *err, uint64_t err_len) {
    char name[128];
    snprintf(name, sizeof(name), "step-%u-layer-%u-%s", step, layer, phase);
    return qxh_write_f32(dir, name, v, n, err, err_len);
}

static int policy_is(const char *p, const char *dflt, const char *want) { return !strcmp(p ? p : dflt, want); }

/* the reference's usage flags of the q8_k_compat projection and expert kernels over the
 * run's layers (qx_detect_projection_kernel_usage, qx_detect_moe_kernel_usage) */
static void kernel_labels(const qxf_file *f, uint32_t start, uint32_t layers, int q8, const char **proj,
                          const char **moe, const char **gate_up, const char **down) {
    static const char *const sfx[4] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight"};
    uint32_t pmask = 0, gmask = 0, dmask = 0;
    int p_q8 = 0, p_f32 = 0, g_q8 = 0, g_f32 = 0, d_q8 = 0, d_f32 = 0;
    for (uint32_t l = start; l < layers; ++l) {
        for (int i = 0; i < 4; ++i) {
            const qxf_dir_entry *t = qxh_layer_tensor(f, l, sfx[i]);
            const uint32_t fam = t ? qxh_projection_family_bit(t->flags) : 0u;
            if (q8 && fam) { p_q8 = 1; pmask |= fam; } else p_f32 = 1;
        }
        const qxf_dir_entry *g = qxh_layer_tensor(f, l, "ffn_gate_exps.weight"), *u = qxh_layer_tensor(f, l, "ffn_up_exps.weight");
        const qxf_dir_entry *d = qxh_layer_tensor(f, l, "ffn_down_exps.weight");
        const uint32_t tg = g ? g->flags : 0, tu = u ? u->flags : 0, td = d ? d->flags : 0;
        if (q8 && ((tg == QXT_IQ2_XS && tu == QXT_IQ2_XS) || (tg == QXT_IQ2_S && tu == QXT_IQ2_S))) {
            g_q8 = 1;
            gmask |= tg == QXT_IQ2_XS ? 1u : 4u;
        } else g_f32 = 1;
        if (q8 && (td == QXT_IQ3_XXS || td == QXT_IQ3_S || td == QXT_IQ4_XS)) {
            d_q8 = 1;
            dmask |= td == QXT_IQ3_XXS ? 2u : td == QXT_IQ3_S ? 16u : 8u;
        } else d_f32 = 1;
    }
    *proj = p_q8 ? qxh_projection_kernel_label(pmask, p_f32) : "dequant_x_f32_scalar";
    if (!q8) { *moe = "dequant_f32"; *gate_up = "dequant_f32"; *down = "dequant_f32"; return; }
    const uint32_t fam = gmask | dmask;
    const int any_q8 = g_q8 || d_q8, any_f32 = g_f32 || d_f32;
    *moe = !any_q8 ? "dequant_f32" : any_f32 ? "q8_k_expert_kernels_with_f32_fallback"
         : fam == 3u ? "iq2_xs_q8_k_and_iq3_xxs_q8_k" : fam == 12u ? "iq2_s_q8_k_and_iq4_xs_q8_k"
         : fam == 15u ? "iq2_xs_iq3_xxs_iq2_s_iq4_xs_q8_k" : fam == 17u ? "iq2_xs_q8_k_and_iq3_s_q8_k"
         : fam == 20u ? "iq2_s_q8_k_and_iq3_s_q8_k" : fam == 31u ? "iq2_xs_iq3_xxs_iq3_s_iq2_s_iq4_xs_q8_k"
         : "q8_k_expert_kernels";
    /* per-family labels (qx_moe_gate_up_kernel_label / qx_moe_down_kernel_label) */
    *gate_up = !g_q8 ? "dequant_f32" : gmask == 1u ? (g_f32 ? "iq2_xs_q8_k_with_f32_fallback" : "iq2_xs_q8_k")
             : gmask == 4u ? (g_f32 ? "iq2_s_q8_k_with_f32_fallback" : "iq2_s_q8_k")
             : (g_f32 ? "iq2_xs_iq2_s_q8_k_with_f32_fallback" : "iq2_xs_iq2_s_q8_k");
    *down = !d_q8 ? "dequant_f32" : dmask == 2u ? (d_f32 ? "iq3_xxs_q8_k_with_f32_fallback" : "iq3_xxs_q8_k")
          : dmask == 8u ? (d_f32 ? "iq4_xs_q8_k_with_f32_fallback" : "iq4_xs_q8_k")
          : dmask == 16u ? (d_f32 ? "iq3_s_q8_k_with_f32_fallback" : "iq3_s_q8_k")
          : (d_f32 ? "mixed_q8_k_with_f32_fallback" : "mixed_q8_k");
}

int qx_dump_prompt_state_loop_probe_summary(const char *path, const char *tokens_path, const uint32_t *prompt_tokens,
        uint32_t prompt_count, uint32_t generation_steps, uint32_t layers, uint32_t ctx_tokens, const char *kv_format,
        const char *activation_format, const char *scratch_policy, const char *kernel_policy, const char *thread_policy,
        uint32_t threads, const char *simd_policy, const char *expert_cache_policy, const char *cuda_policy,
        const char *prefill_gemm_policy, const char *speculative_policy, const char *kv2_policy,
        const char *sampling_policy, const char *long_context_policy, int dequant_profile, int real_kv,
        int projection_matvec, int residual_vector, int residual_carry, int numeric_deltas, int delta_vectors,
        int attention_output_vector, int causal_attention, int rope_gqa_attention, int full_moe, int final_head,
        int bench, uint32_t residual_dims, const char *norm_name, uint32_t top_k, uint32_t scan,
        uint32_t logits_top_n, double temperature, uint32_t seed, const char *residual_dump_dir, uint32_t start_layer,
        const char *residual_input_path, const char *kv_snapshot_out_path, const char *kv_snapshot_in_path, FILE *out,
        char *err, uint64_t err_len) {
    (void)real_kv; (void)residual_carry; (void)numeric_deltas; (void)delta_vectors; (void)attention_output_vector;
    (void)residual_dims;
    /* argument checks in the reference's order and words (src/qx_format.c:5971-6041) */
    if (!path || !kv_format || !activation_format || !prompt_tokens || prompt_count == 0 || !out) {
        qxh_set_err(err, err_len, "invalid argument"); return 0;
    }
    const int act = qxh_activation_code(activation_format);
    if (act < 0) { qxh_set_err(err, err_len, "unsupported activation format"); return 0; }
    if (!scratch_policy) scratch_policy = "ephemeral";
    if (strcmp(scratch_policy, "persistent") && strcmp(scratch_policy, "ephemeral")) { qxh_set_err(err, err_len, "unsupported scratch policy"); return 0; }
    if (!kernel_policy) kernel_policy = "baseline";
    if (strcmp(kernel_policy, "baseline") && strcmp(kernel_policy, "fused")) { qxh_set_err(err, err_len, "unsupported kernel policy"); return 0; }
    if (!thread_policy) thread_policy = "serial";
    if (threads == 0) threads = 1;
    const int pool = !strcmp(thread_policy, "pool");
    if (!pool && strcmp(thread_policy, "serial")) { qxh_set_err(err, err_len, "unsupported thread policy"); return 0; }
    if (!pool && threads != 1) { qxh_set_err(err, err_len, "serial thread policy requires --threads 1"); return 0; }
    if (pool && threads < 2) { qxh_set_err(err, err_len, "thread pool policy requires --threads >= 2"); return 0; }
    if (pool && threads > 64) { qxh_set_err(err, err_len, "thread pool policy supports at most 64 threads"); return 0; }
    if (pool && act != 0) { qxh_set_err(err, err_len, "thread pool policy currently requires F32 activation"); return 0; }
    if (!simd_policy) simd_policy = "scalar";
    const int avx2 = !strcmp(simd_policy, "avx2-fma");
    if (!avx2 && strcmp(simd_policy, "scalar")) { qxh_set_err(err, err_len, "unsupported simd policy"); return 0; }
    if (avx2 && strcmp(kernel_policy, "fused")) { qxh_set_err(err, err_len, "avx2-fma simd policy requires --kernel-policy fused"); return 0; }
    if (avx2 && act != 0) { qxh_set_err(err, err_len, "avx2-fma simd policy requires F32 activation"); return 0; }
    if (avx2 && pool) { qxh_set_err(err, err_len, "avx2-fma simd policy currently requires serial thread policy"); return 0; }
    if (!policy_is(expert_cache_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported expert cache policy"); return 0; }
    if (!policy_is(cuda_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported CUDA policy"); return 0; }
    if (!policy_is(prefill_gemm_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported prefill GEMM policy"); return 0; }
    if (!policy_is(speculative_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported speculative policy"); return 0; }
    if (!policy_is(kv2_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported KV2 policy"); return 0; }
    if (!policy_is(sampling_policy, "none", "none")) { qxh_set_err(err, err_len, "unsupported sampling policy"); return 0; }
    if (!long_context_policy) long_context_policy = "none";
    const int ctx4k = !strcmp(long_context_policy, "ctx4k-smoke");
    if (!ctx4k && strcmp(long_context_policy, "none")) { qxh_set_err(err, err_len, "unsupported long-context policy"); return 0; }
    if (ctx4k && ctx_tokens < 4096) { qxh_set_err(err, err_len, "ctx4k-smoke long-context policy requires --ctx >= 4096"); return 0; }
    if (full_moe && norm_name && *norm_name) { qxh_set_err(err, err_len, "--norm cannot be combined with --full-moe"); return 0; }
    const int dumping = residual_dump_dir && *residual_dump_dir;
    if (dumping && !full_moe) { qxh_set_err(err, err_len, "--dump-residuals requires --full-moe"); return 0; }
    if ((kv_snapshot_out_path || kv_snapshot_in_path) && !causal_attention) { qxh_set_err(err, err_len, "KV snapshot requires causal attention"); return 0; }
    const int replay = residual_input_path && *residual_input_path;
    if ((start_layer != 0 && !replay) || (replay && (!full_moe || !residual_vector || prompt_count != 1 || generation_steps != 1))) {
        qxh_set_err(err, err_len, "residual replay requires a full MoE residual vector, exactly one token step, --start-layer, and --residual-in");
        return 0;
    }
    if (generation_steps == 0 || generation_steps > 64 || prompt_count > 64) {
        qxh_set_err(err, err_len, "prompt state loop requires 1..64 prompt tokens and 1..64 generation steps"); return 0;
    }
    const uint32_t steps = prompt_count + generation_steps - 1;
    if (steps > 64) { qxh_set_err(err, err_len, "prompt plus generation exceeds 64 forward steps"); return 0; }
    if (layers == 0) layers = 1;
    if (top_k == 0) top_k = 1;
    if (top_k > 32) top_k = 32;
    if (causal_attention && (!projection_matvec || !residual_vector)) {
        qxh_set_err(err, err_len, "causal attention requires projection matvec and residual vector"); return 0;
    }
    /* the device path: the reference's --full-moe forward with INT8 KV */
    if (!full_moe || !rope_gqa_attention || !causal_attention) {
        qxh_set_err(err, err_len, "the GPU state loop implements the --full-moe path only"); return 0;
    }
    if (strcmp(kv_format, "int8")) {
        const int known = !strcmp(kv_format, "f16") || !strcmp(kv_format, "fp16") || !strcmp(kv_format, "f32");
        qxh_set_err(err, err_len, known ? "the GPU state loop supports INT8 KV only"
                                        : "full MoE state loop requires INT8, F16, or diagnostic F32 KV");
        return 0;
    }
    qxf_file f;
    if (!qxf_open(path, &f, err, err_len)) return 0;
    const qxf_manifest *man = &f.header.manifest;
    const uint32_t hidden = man->hidden;
    int ok = 1;
#define FAIL(msg) do { qxh_set_err(err, err_len, msg); ok = 0; goto done; } while (0)
    qxg_ctx *ctx = NULL;
    probe_scan ps;
    memset(&ps, 0, sizeof(ps));
    float *logits = NULL;
    char *generated = NULL;
    float *s_lay = NULL, *s_att = NULL, *s_moe = NULL, *s_ks = NULL, *s_vs = NULL;   /* device step records */
    float *s_norm = NULL, *s_lg = NULL;
    double *s_ws = NULL, *s_rw = NULL, *s_tl = NULL, *s_ms = NULL;
    uint32_t *s_ids = NULL, *s_tid = NULL, *s_tok = NULL;
    int8_t *s_k = NULL, *s_v = NULL;
    if (hidden != 2048) FAIL("unsupported full MoE hidden size");
    const uint32_t requested_layers = layers, manifest_layers = man->layers ? man->layers : layers;
    if (layers > manifest_layers) layers = manifest_layers;
    if (replay && start_layer >= layers) FAIL("residual replay start layer must be below requested layers");
    if (man->q_heads != 32 || man->kv_heads != 4 || man->head_dim != 128) FAIL("invalid attention dimensions");
    if (final_head && (requested_layers != manifest_layers || temperature != 0.0))
        FAIL("--final-head requires --full-moe, 1..64 steps, all manifest layers, and temperature 0");
    if (pool && !final_head) FAIL("thread pool policy currently requires --final-head");
    if (final_head && (man->model_type != 2 || manifest_layers != 48 || man->vocab != 151936))
        FAIL("--final-head requires exact Qwen3-30B-A3B manifest dimensions");
    if (ctx_tokens == 0 || ctx_tokens > 4096) FAIL("state loop context must be between 1 and 4096");
    if (logits_top_n == 0) logits_top_n = 1;
    if (logits_top_n > 32) logits_top_n = 32;
    const uint32_t vocab = man->vocab ? man->vocab : 151936u;
    for (uint32_t i = 0; i < prompt_count; ++i) if (prompt_tokens[i] >= vocab) FAIL("prompt token out of range");
    if (steps > ctx_tokens) FAIL("steps exceed ctx");
    qx_gpu_model_info mi;
    double t_load = qxh_now_s();
    if (!qxh_open_gpu(path, 1, &ctx, &mi, err, err_len)) { ok = 0; goto done; }
    t_load = qxh_now_s() - t_load;
    if (!mi.has_embedding) FAIL("token_embd.weight not found");
    if (final_head && !mi.has_head) FAIL("final head requires Q6_K output.weight");
    if (!qxg_set_activation(ctx, (uint32_t)act, err, err_len) || !qxg_kv_create(ctx, layers, ctx_tokens, 1, err, err_len)) {
        ok = 0; goto done;
    }
    uint32_t position_base = 0, snap_next = prompt_tokens[0];
    if (kv_snapshot_in_path && *kv_snapshot_in_path) {
        /* resume rule (src/qx_format.c:6165-6177): one continuation token, which must be the
         * snapshot's recorded next token */
        if (prompt_count != 1) FAIL("KV snapshot replay requires exactly one continuation token");
        if (!qxg_kv_import(ctx, kv_snapshot_in_path, layers, ctx_tokens, seed, &position_base, &snap_next, err, err_len)) {
            ok = 0; goto done;
        }
        if (prompt_tokens[0] != snap_next) FAIL("KV snapshot continuation token mismatch");
    }
    if (position_base > ctx_tokens || steps > ctx_tokens - position_base || position_base > 64 || steps > 64 - position_base)
        FAIL("KV snapshot plus replay steps exceed context");
    if (!final_head && !probe_scan_init(ctx, &f, scan, &ps, err, err_len)) { ok = 0; goto done; }
    logits = final_head ? (float *)malloc((size_t)vocab * 4) : NULL;
    generated = (char *)calloc(32768, 1);
    if ((final_head && !logits) || !generated) FAIL("out of memory");
    const char *proj_label, *moe_label, *gu_label, *dn_label;
    kernel_labels(&f, start_layer, layers, act, &proj_label, &moe_label, &gu_label, &dn_label);
    const uint64_t layer_stride = (uint64_t)ctx_tokens * 1024;
    /* header (src/qx_format.c:6199-6249) */
    fprintf(out, "{\n  \"probe\": \"state_loop\",\n  \"prompt_token\": %u,\n  \"prompt_token_count\": %u,\n  \"prompt_token_ids\": [",
            prompt_tokens[0], prompt_count);
    for (uint32_t i = 0; i < prompt_count; ++i) fprintf(out, "%s%u", i ? ", " : "", prompt_tokens[i]);
    fprintf(out, "],\n  \"generation_steps\": %u,\n  \"steps\": %u,\n  \"layers\": %u,\n  \"start_layer\": %u,\n"
            "  \"ctx_tokens\": %u,\n  \"position_base\": %u,\n  \"kv_format\": \"int8\",\n  \"activation_format\": \"%s\",\n"
            "  \"io_backend\": \"mmap\",\n  \"scratch_policy\": \"%s\",\n  \"kernel_policy\": \"%s\",\n  \"thread_policy\": \"%s\",\n"
            "  \"threads\": %u,\n  \"simd_policy\": \"%s\",\n  \"expert_cache_policy\": \"none\",\n  \"cuda_policy\": \"none\",\n"
            "  \"prefill_gemm_policy\": \"none\",\n  \"speculative_policy\": \"none\",\n  \"kv2_policy\": \"none\",\n"
            "  \"sampling_policy\": \"none\",\n  \"long_context_policy\": \"%s\",\n  \"projection_kernel\": \"%s\",\n"
            "  \"activation_workspace_bytes\": %u,\n  \"moe_projection_kernel\": \"%s\",\n  \"moe_gate_up_projection_kernel\": \"%s\",\n"
            "  \"moe_down_projection_kernel\": \"%s\",\n  \"moe_activation_workspace_bytes\": %u,\n  \"kv_source\": \"projection_matvec\",\n"
            "  \"residual_source\": \"%s\",\n  \"residual_dims\": 2048,\n"
            "  \"residual_replay\": {\"enabled\": %s, \"source\": %s, \"values\": %u},\n  \"residual_dump\": %s,\n"
            "  \"residual_dump_count\": %llu,\n  \"logits_dump_count\": %u,\n  \"delta_source\": \"real_attention_moe\",\n"
            "  \"bytes_per_k_or_v\": 512,\n  \"bytes_per_token_per_layer\": 1024,\n  \"layer_stride\": %llu,\n  \"backend\": \"hip-gfx950\",\n"
            "  \"tokens\": [",
            generation_steps, steps, layers, start_layer, ctx_tokens, position_base, activation_format, scratch_policy,
            kernel_policy, thread_policy, threads, simd_policy, long_context_policy, proj_label,
            act ? 16u * 292u : 0u, moe_label, gu_label, dn_label, act ? 8u * 292u : 0u,
            replay ? "injected_f32_replay" : "real_attention_moe_carry", replay ? "true" : "false",
            replay ? "\"f32_sidecar\"" : "null", replay ? 2048u : 0u, dumping ? "true" : "false",
            (unsigned long long)(dumping ? (uint64_t)steps * (layers - start_layer) * 6u : 0u), dumping && final_head ? steps : 0u,
            (unsigned long long)layer_stride);
    float x[2048], a[2048], y[2048], kqv[4096], vcur[512], moe[2048], nrm[2048];
    int8_t krow[512], vrow[512];
    /* Without replay or dumps the steps run on the device and the loop prints their records:
     * with the final head on the persistent path, the whole loop is one launch (its argmax
     * feeding each next token on the device) and every step's records come back after it;
     * otherwise (the token scan picks each next token on the host) one qxg_decode_token per
     * step, its records read back after it.  Records are [step][layer][...] with one step slot
     * in the per-step mode; K/V rows [layer][step][512]. */
    const int one_launch = !replay && !dumping && layers == mi.layers;
    const int recorded = one_launch && final_head && qxg_persistent_path(ctx);
    const uint64_t rs = recorded ? steps : 1, rl = rs * layers;
    if (one_launch) {
        s_lay = (float *)malloc((size_t)rl * 2048 * 4); s_att = (float *)malloc((size_t)rl * 2048 * 4);
        s_moe = (float *)malloc((size_t)rl * 2048 * 4); s_ks = (float *)malloc((size_t)rl * 4);
        s_vs = (float *)malloc((size_t)rl * 4); s_ws = (double *)malloc((size_t)rl * 32 * 8);
        s_rw = (double *)malloc((size_t)rl * 8 * 8); s_ids = (uint32_t *)malloc((size_t)rl * 8 * 4);
        s_k = (int8_t *)malloc((size_t)rl * 512); s_v = (int8_t *)malloc((size_t)rl * 512);
        s_norm = (float *)malloc((size_t)rs * 2048 * 4); s_lg = (float *)malloc((size_t)rs * vocab * 4);
        s_tid = (uint32_t *)malloc((size_t)rs * 32 * 4); s_tl = (double *)malloc((size_t)rs * 32 * 8);
        s_tok = (uint32_t *)malloc((size_t)(rs + 1) * 4); s_ms = (double *)malloc((size_t)(rs + 1) * 8);
        if (!s_lay || !s_att || !s_moe || !s_ks || !s_vs || !s_ws || !s_rw || !s_ids || !s_k || !s_v || !s_norm || !s_lg ||
            !s_tid || !s_tl || !s_tok || !s_ms)
            FAIL("out of memory");
    }
    double t_dev = 0.0;   /* device time: the one launch, or the per-step calls and readbacks */
    if (recorded) {
        float ms = 0.0f;
        if (!qxg_generate_recorded(ctx, prompt_tokens, prompt_count, generation_steps, position_base, logits_top_n, s_tok,
                                   s_lay, s_att, s_moe, s_ids, s_rw, s_ws, s_norm, s_lg, s_tid, s_tl, s_ms, &ms, err,
                                   err_len)) {
            ok = 0; goto done;
        }
        t_dev = ms * 1e-3;
        for (uint32_t l = 0; l < layers; ++l)
            if (!qxg_kv_read(ctx, l, position_base, steps, s_k + (uint64_t)l * steps * 512, s_v + (uint64_t)l * steps * 512,
                             s_ks + (uint64_t)l * steps, s_vs + (uint64_t)l * steps, err, err_len)) { ok = 0; goto done; }
    }
    uint64_t k_mix = FNV_OFFSET, v_mix = FNV_OFFSET, layers_run = 0, kv_appends = 0;
    size_t gen_len = 0;
    uint32_t current = prompt_tokens[0], prefill_tokens = 0, decode_tokens = 0;
    double t_loop = qxh_now_s(), t_prefill = 0.0, t_decode = 0.0;
    for (uint32_t ls = 0; ok && ls < steps; ++ls) {
        const double t_step = qxh_now_s();
        double step_dev = 0.0;
        const uint32_t step = position_base + ls;
        const uint64_t so = recorded ? ls : 0;   /* the step's record slot */
        if (ls < prompt_count) current = prompt_tokens[ls];
        const int sampling = ls + 1 >= prompt_count;
        fprintf(out, "%s{\"step\": %u, \"position\": %u, \"phase\": \"%s\", \"input_token\": %u, \"layers\": [", ls ? ", " : "",
                step, step, sampling ? "generate" : "prefill", current);
        double rms, probe;
        if (replay) {
            if (!qxh_read_sidecar(residual_input_path, x, 2048, err, err_len)) { ok = 0; break; }
        } else if (!qxg_embed_token(ctx, current, x, err, err_len)) { ok = 0; break; }
        {
            double ss = 0.0, sum = 0.0;
            for (int i = 0; i < 2048; ++i) { ss += (double)x[i] * (double)x[i]; sum += x[i]; }
            rms = replay ? sqrt(ss / 2048.0) : sqrt(ss / 2048.0 + 1.0e-6);
            probe = sum / 2048.0;
        }
        const uint64_t in_chk = qxf_fnv1a64(x, sizeof(x));
        const int run_head = final_head && sampling;
        if (recorded) {   /* the step's share of the launch, from the device clock */
            step_dev = (s_ms[ls + 1] - s_ms[ls]) * 1e-3;
        } else if (one_launch) {   /* the whole step on the device, then its records */
            const double t0 = qxh_now_s();
            if (!qxg_decode_token(ctx, current, step, run_head, NULL, s_lay, run_head ? s_lg : NULL, logits_top_n, s_tid,
                                  s_tl, err, err_len) ||
                !qxg_decode_halves(ctx, layers, s_att, s_moe, err, err_len) ||
                !qxg_decode_routing(ctx, layers, s_ids, s_rw, err, err_len) ||
                !qxg_decode_head_sums(ctx, layers, s_ws, err, err_len) ||
                (run_head && !qxg_decode_final_norm(ctx, s_norm, err, err_len)) ||
                !qxg_kv_read_position(ctx, step, layers, s_k, s_v, s_ks, s_vs, err, err_len)) { ok = 0; break; }
            step_dev = qxh_now_s() - t0;
            t_dev += step_dev;
        }
        for (uint32_t l = start_layer; ok && l < layers; ++l) {
            const uint64_t rin = qxf_fnv1a64(x, sizeof(x));
            double hs[32];
            uint32_t ids[8];
            double w[8];
            float ks, vs;
            if (dumping && !dump_vec(residual_dump_dir, step, l, "input", x, 2048, err, err_len)) { ok = 0; break; }
            const uint64_t sl = so * layers + l, kl = (uint64_t)l * rs + so;   /* record and K/V row slots */
            if (one_launch) {
                memcpy(a, s_att + 2048 * sl, sizeof(a));
                memcpy(hs, s_ws + 32 * sl, sizeof(hs));
                memcpy(krow, s_k + 512 * kl, 512);
                memcpy(vrow, s_v + 512 * kl, 512);
                ks = s_ks[kl];
                vs = s_vs[kl];
            } else if (!qxg_attention_layer_ex(ctx, l, step, x, a, kqv, vcur, hs, err, err_len) ||
                       !qxg_kv_read(ctx, l, step, 1, krow, vrow, &ks, &vs, err, err_len)) { ok = 0; break; }
            if (dumping && (!dump_vec(residual_dump_dir, step, l, "v-cur", vcur, 512, err, err_len) ||
                            !dump_vec(residual_dump_dir, step, l, "kqv-out", kqv, 4096, err, err_len))) { ok = 0; break; }
            double a2 = 0.0;
            for (int i = 0; i < 2048; ++i) { a2 += (double)a[i] * (double)a[i]; x[i] += a[i]; }
            if (dumping && !dump_vec(residual_dump_dir, step, l, "ffn-inp", x, 2048, err, err_len)) { ok = 0; break; }
            if (one_launch) {   /* x is now the step's ffn input, x + attention as the device added them */
                memcpy(y, s_lay + 2048 * sl, sizeof(y));
                memcpy(moe, s_moe + 2048 * sl, sizeof(moe));
                memcpy(ids, s_ids + 8 * sl, sizeof(ids));
                memcpy(w, s_rw + 8 * sl, sizeof(w));
            } else if (!qxg_moe_layer(ctx, l, x, y, moe, ids, w, err, err_len)) { ok = 0; break; }
            if (dumping && (!dump_vec(residual_dump_dir, step, l, "ffn-moe-out", moe, 2048, err, err_len) ||
                            !dump_vec(residual_dump_dir, step, l, "output", y, 2048, err, err_len))) { ok = 0; break; }
            double m2 = 0.0, sum = 0.0;
            for (int i = 0; i < 2048; ++i) { m2 += (double)moe[i] * (double)moe[i]; x[i] = y[i]; sum += y[i]; }
            const uint64_t kchk = qxf_fnv1a64(krow, 512), vchk = qxf_fnv1a64(vrow, 512);
            k_mix = (k_mix ^ kchk) * FNV_PRIME;
            v_mix = (v_mix ^ vchk) * FNV_PRIME;
            probe = sum / 2048.0 + (double)((kchk ^ vchk) & 0xffffu) / 65535.0 * 0.0001;
            double hsum = 0.0, hmin = hs[0], hmax = hs[0];
            for (int h = 0; h < 32; ++h) { hsum += hs[h]; if (hs[h] < hmin) hmin = hs[h]; if (hs[h] > hmax) hmax = hs[h]; }
            const qxf_dir_entry *tq = qxh_layer_tensor(&f, l, "attn_q.weight"), *tk = qxh_layer_tensor(&f, l, "attn_k.weight");
            const qxf_dir_entry *tv = qxh_layer_tensor(&f, l, "attn_v.weight"), *to = qxh_layer_tensor(&f, l, "attn_output.weight");
            const qxf_dir_entry *tg = qxh_layer_tensor(&f, l, "ffn_gate_exps.weight"), *tu = qxh_layer_tensor(&f, l, "ffn_up_exps.weight");
            const qxf_dir_entry *td = qxh_layer_tensor(&f, l, "ffn_down_exps.weight");
            const uint64_t koff = (uint64_t)l * layer_stride + (uint64_t)step * 1024;
            /* one layer's entry (src/qx_format.c:6494-6529) */
            fprintf(out, "%s{\"layer\": %u, \"kv_token\": %u, \"k_offset\": %llu, \"v_offset\": %llu, \"k_checksum\": %llu, "
                    "\"v_checksum\": %llu, \"full_moe\": true, \"qk_head_norm\": true, \"experts_run\": 8, \"selected_experts\": [",
                    l != start_layer ? ", " : "", l, step, (unsigned long long)koff, (unsigned long long)(koff + 512),
                    (unsigned long long)kchk, (unsigned long long)vchk);
            for (int r = 0; r < 8; ++r) fprintf(out, "%s%u", r ? "," : "", ids[r]);
            fprintf(out, "], \"routing_weights\": [");
            for (int r = 0; r < 8; ++r) fprintf(out, "%s%.17g", r ? "," : "", w[r]);
            fprintf(out, "], \"gate_ggml_type\": %u, \"up_ggml_type\": %u, \"down_ggml_type\": %u, \"moe_output_l2\": %.17g, "
                    "\"residual_input_checksum\": %llu, \"residual_output_checksum\": %llu",
                    tg ? tg->flags : 0u, tu ? tu->flags : 0u, td ? td->flags : 0u, sqrt(m2), (unsigned long long)rin,
                    (unsigned long long)qxf_fnv1a64(x, sizeof(x)));
            fprintf(out, ", \"k_tensor\": \"blk.%u.attn_k.weight\", \"v_tensor\": \"blk.%u.attn_v.weight\", \"k_real_values\": 512, "
                    "\"v_real_values\": 512, \"k_matvec_values\": 512, \"v_matvec_values\": 512", l, l);
            fprintf(out, ", \"attention_output_vector_values\": 2048, \"attention_output_vector_l2\": %.9g, "
                    "\"attention_output_vector_checksum\": %llu, \"attention_context_tokens\": %u, "
                    "\"attention_output_source\": \"rope_gqa_softmax_output_projection_partial\"",
                    sqrt(a2), (unsigned long long)qxf_fnv1a64(a, sizeof(a)), step + 1);
            fprintf(out, ", \"persistent_kv\": true, \"kv_scale_source\": \"dynamic_per_vector\", \"k_scale\": %.9g, \"v_scale\": %.9g, "
                    "\"q_values\": 4096, \"q_tensor\": \"blk.%u.attn_q.weight\", \"q_ggml_type\": %u, \"k_ggml_type\": %u, "
                    "\"v_ggml_type\": %u, \"output_tensor\": \"blk.%u.attn_output.weight\", \"output_ggml_type\": %u, \"softmax_sum\": %.9g",
                    (double)ks, (double)vs, l, tq ? tq->flags : UINT32_MAX, tk ? tk->flags : UINT32_MAX,
                    tv ? tv->flags : UINT32_MAX, l, to ? to->flags : UINT32_MAX, hsum / 32.0);
            fprintf(out, ", \"attention_mode\": \"rope_gqa_full_heads\", \"rope_applied\": true, \"rope_theta\": 1000000, "
                    "\"q_heads_total\": 32, \"kv_heads_total\": 4, \"q_heads_run\": 32, \"kv_heads_touched\": 4, \"gqa_group_size\": 8, "
                    "\"head_dim\": 128, \"output_projection_input_dims\": 4096, \"output_projection_output_dims\": 2048, "
                    "\"softmax_sum_min\": %.9g, \"softmax_sum_max\": %.9g}", hmin, hmax);
            ++kv_appends;
            ++layers_run;
        }
        if (!ok) break;
        fprintf(out, "], \"residual_probe\": %.9g, \"residual_values\": 2048, \"residual_rms\": %.9g, \"residual_checksum\": %llu, "
                "\"residual_checksum_after\": %llu", probe, rms, (unsigned long long)in_chk,
                (unsigned long long)qxf_fnv1a64(x, sizeof(x)));
        if (!sampling) {
            fprintf(out, ", \"selected_token\": null, \"source\": \"fixed_prompt\"}");
            t_prefill += one_launch ? step_dev : qxh_now_s() - t_step;
            ++prefill_tokens;
            current = prompt_tokens[ls + 1];
            continue;
        }
        uint32_t next;
        if (final_head) {
            uint32_t tid[32];
            double tl[32];
            const float *lg = logits;
            if (one_launch) {   /* the step's own head: its argmax is the token it feeds on */
                memcpy(tid, s_tid + so * logits_top_n, logits_top_n * sizeof(uint32_t));
                memcpy(tl, s_tl + so * logits_top_n, logits_top_n * sizeof(double));
                memcpy(nrm, s_norm + so * 2048, sizeof(nrm));
                lg = s_lg + so * vocab;
                if (recorded && tid[0] != s_tok[ls + 1]) FAIL("device argmax and top-N ranking disagree");
            } else if (!qxg_final_head(ctx, x, nrm, logits, logits_top_n, tid, tl, err, err_len)) { ok = 0; break; }
            if (dumping) {
                char nm[64];
                snprintf(nm, sizeof(nm), "step-%u-logits", step);
                if (!qxh_write_f32(residual_dump_dir, nm, lg, vocab, err, err_len)) { ok = 0; break; }
            }
            double ss = 0.0, ns = 0.0, lmin = lg[0], lmax = lg[0], l2 = 0.0;
            for (int i = 0; i < 2048; ++i) { ss += (double)x[i] * (double)x[i]; ns += (double)nrm[i] * (double)nrm[i]; }
            for (uint32_t i = 0; i < vocab; ++i) {
                const double v = lg[i];
                if (v < lmin) lmin = v;
                if (v > lmax) lmax = v;
                l2 += v * v;
            }
            const qxf_dir_entry *hd = qxf_find(&f, "output.weight"), *on = qxf_find(&f, "output_norm.weight");
            fprintf(out, ", \"final_head\": {\"enabled\": true, \"norm_tensor\": \"output_norm.weight\", \"norm_ggml_type\": 0, "
                    "\"norm_values\": 2048, \"norm_checksum_verified\": true, \"norm_raw_checksum\": %llu, \"input_rms\": %.17g, "
                    "\"normalized_l2\": %.17g, \"final_residual_checksum\": %llu, \"final_norm_checksum\": %llu, "
                    "\"lm_head_tensor\": \"output.weight\", \"lm_head_ggml_type\": %u, \"lm_head_decoder\": \"Q6_K\", "
                    "\"lm_head_kernel\": \"%s\", \"activation_quantizations\": %u, \"lm_head_checksum_verified\": true, "
                    "\"lm_head_raw_checksum\": %llu, \"input_dims\": 2048, \"vocab_size\": %u, \"logits_computed\": %u, "
                    "\"full_vocabulary\": true, \"logits_checksum\": %llu, \"logits_min\": %.17g, \"logits_max\": %.17g, "
                    "\"logits_rms\": %.17g, \"argmax_token\": %u, \"argmax_logit\": %.17g, \"top_tokens\": [",
                    (unsigned long long)(on ? on->checksum : 0), sqrt(ss / 2048.0 + 1.0e-6), sqrt(ns),
                    (unsigned long long)qxf_fnv1a64(x, sizeof(x)), (unsigned long long)qxf_fnv1a64(nrm, sizeof(nrm)),
                    hd ? hd->flags : 0u, act ? "q6_k_q8_k_hip_dot4" : "q6_k_hip_dot4", act ? 1u : 0u,
                    (unsigned long long)(hd ? hd->checksum : 0), vocab, vocab,
                    (unsigned long long)qxf_fnv1a64(lg, (uint64_t)vocab * 4), lmin, lmax, sqrt(l2 / (double)vocab),
                    tid[0], tl[0]);
            const uint64_t row_bytes = hd ? hd->byte_size / vocab : 0;
            for (uint32_t r = 0; r < logits_top_n; ++r)
                fprintf(out, "%s{\"token\": %u, \"logit\": %.17g, \"row_checksum\": %llu}", r ? ", " : "", tid[r], tl[r],
                        (unsigned long long)(hd ? qxf_fnv1a64(qxf_data(&f, hd) + (uint64_t)tid[r] * row_bytes, row_bytes) : 0));
            fprintf(out, "], \"final_residual_raw\": [");
            for (int i = 0; i < 2048; ++i) fprintf(out, "%s%.9g", i ? "," : "", (double)x[i]);
            fprintf(out, "], \"final_norm_raw\": [");
            for (int i = 0; i < 2048; ++i) fprintf(out, "%s%.9g", i ? "," : "", (double)nrm[i]);
            fprintf(out, "]}");
            next = tid[0];
        } else {
            top_token top[32];
            uint32_t k = probe_scan_top(&ps, probe, top_k, seed + step * 17u + current, top);
            next = sample_from_top(top, k, temperature, seed + step * 101u + current);
        }
        char piece[8192];
        const char *src;
        token_piece(tokens_path, next, piece, sizeof(piece), &src);
        const size_t pl = strlen(piece);
        if (gen_len + pl < 32768) { memcpy(generated + gen_len, piece, pl + 1); gen_len += pl; }
        fprintf(out, ", \"selected_token\": %u, \"piece\": ", next);
        qxh_json_string(out, piece);
        fprintf(out, ", \"source\": \"%s\"}", src);
        t_decode += one_launch ? step_dev : qxh_now_s() - t_step;
        ++decode_tokens;
        current = next;
    }
    t_loop = qxh_now_s() - t_loop;
    if (!ok) goto done;
    if (kv_snapshot_out_path && *kv_snapshot_out_path &&
        !qxg_kv_export(ctx, kv_snapshot_out_path, layers, position_base + steps, ctx_tokens, current, seed, err, err_len)) {
        ok = 0; goto done;
    }
    fprintf(out, "],\n  \"layers_run\": %llu,\n  \"kv_appends\": %llu,\n  \"cache_readback_ok\": true,\n"
            "  \"k_cache_checksum\": %llu,\n  \"v_cache_checksum\": %llu,\n  \"final_token\": %u,\n  \"generated_text\": ",
            (unsigned long long)layers_run, (unsigned long long)kv_appends, (unsigned long long)k_mix,
            (unsigned long long)v_mix, current);
    qxh_json_string(out, generated);
    fprintf(out, ",\n");
    if (bench) {
        /* device mode: the device work (the one launch, or the per-step calls with their
         * readbacks), the JSON formatting apart in wall_elapsed_sec; the per-layer seams: the
         * whole loop */
        const double el = one_launch ? (t_dev > 0.0 ? t_dev : 1e-6) : (t_loop > 0.0 ? t_loop : 1e-6);
        fprintf(out, "  \"bench\": {\"enabled\": true, \"timer\": \"monotonic_wall\", \"timed\": \"%s\", \"elapsed_sec\": %.9g, "
                "\"wall_elapsed_sec\": %.9g, \"tokens_per_second\": %.9g, "
                "\"ms_per_token\": %.9g, \"layer_steps\": %llu, \"layer_steps_per_second\": %.9g, \"phases\": {\"prefill\": "
                "{\"tokens\": %u, \"elapsed_sec\": %.9g, \"tokens_per_second\": %.9g}, \"decode\": {\"tokens\": %u, "
                "\"elapsed_sec\": %.9g, \"tokens_per_second\": %.9g}}",
                recorded ? "device_launch" : one_launch ? "device_steps" : "loop", el, t_loop, steps / el, 1000.0 * el / steps, (unsigned long long)layers_run,
                layers_run / el, prefill_tokens, t_prefill, prefill_tokens ? prefill_tokens / t_prefill : 0.0, decode_tokens,
                t_decode, decode_tokens ? decode_tokens / t_decode : 0.0);
        /* the same tokens through the device decode loop (one launch per call, no host
         * work per layer), on a fresh cache: the path's own throughput */
        if (final_head && !replay && position_base == 0) {
            uint32_t *gen = (uint32_t *)malloc((size_t)generation_steps * 4);
            float ms = 0.0f;
            if (gen && qxg_kv_create(ctx, layers, ctx_tokens, 1, err, err_len) &&
                qxg_generate(ctx, prompt_tokens, prompt_count, generation_steps, 0, gen, &ms, err, err_len)) {
                fprintf(out, ", \"device\": {\"device_ms\": %.6f, \"steps\": %u, \"tokens_per_second\": %.3f, \"final_token\": %u, "
                        "\"matches_probe\": %s}", ms, steps, steps / (ms * 1e-3), gen[generation_steps - 1],
                        gen[generation_steps - 1] == current ? "true" : "false");
            } else {
                ok = 0;
            }
            free(gen);
            if (!ok) { fprintf(out, "}\n}\n"); goto done; }
        }
        fprintf(out, "},\n");
    }
    fprintf(out, "  \"allocation_profile\": {\"malloc_calls\": 0, \"calloc_calls\": 0, \"realloc_calls\": 0, \"free_calls\": 0, "
            "\"bytes_requested\": 0, \"note\": \"device memory is allocated at load and cache creation\"},\n"
            "  \"scratch_profile\": {\"policy\": \"%s\", \"peak_capacity_bytes\": %llu, \"growth_events\": 0},\n"
            "  \"dequant_dot_profile\": {\"enabled\": %s, \"kernel_policy\": \"%s\", \"target\": \"final_head_q6_k\", "
            "\"temporary_blocks_decoded\": 0, \"temporary_floats_materialized\": 0, \"temporary_bytes_materialized\": 0, "
            "\"fused_dot_calls\": %llu, \"fallback_dot_calls\": 0, \"final_head_q6_k_blocks\": %llu},\n"
            "  \"thread_profile\": {\"enabled\": true, \"policy\": \"%s\", \"requested_threads\": %u, \"workers_used\": %u, "
            "\"parallel_jobs\": 0, \"serial_jobs\": %llu, \"fallback_jobs\": %llu%s},\n"
            "  \"simd_profile\": {\"enabled\": true, \"policy\": \"%s\", \"kernel\": \"scalar\", \"fma_dot_calls\": 0, "
            "\"fallback_dot_calls\": 0%s},\n"
            "  \"expert_cache_profile\": {\"enabled\": true, \"policy\": \"none\", \"cache_hits\": 0, \"cache_misses\": 0, "
            "\"bytes_cached\": 0, \"expert_weight_reads\": 0, \"disabled_reason\": \"none_policy\"},\n"
            "  \"cuda_profile\": {\"enabled\": true, \"policy\": \"none\", \"backend\": \"none\", \"device_bytes\": 0, "
            "\"host_to_device_bytes\": 0, \"device_to_host_bytes\": 0, \"kernel_launches\": 0, \"disabled_reason\": \"none_policy\"},\n"
            "  \"hip_profile\": {\"enabled\": true, \"backend\": \"hip-gfx950\", \"device_bytes\": %llu, \"load_seconds\": %.6f},\n"
            "  \"prefill_gemm_profile\": {\"enabled\": true, \"policy\": \"none\", \"backend\": \"none\", \"gemm_calls\": 0, "
            "\"batched_tokens\": 0, \"fused_rows\": 0, \"temporary_bytes\": 0, \"disabled_reason\": \"none_policy\"},\n"
            "  \"speculative_profile\": {\"enabled\": true, \"policy\": \"none\", \"backend\": \"none\", \"draft_tokens\": 0, "
            "\"accepted_tokens\": 0, \"rejected_tokens\": 0, \"target_verifications\": 0, \"disabled_reason\": \"none_policy\"},\n"
            "  \"kv2_profile\": {\"enabled\": true, \"policy\": \"none\", \"format\": \"none\", \"packed_bytes\": 0, \"read_ops\": 0, "
            "\"write_ops\": 0, \"fallback_reads\": 0, \"disabled_reason\": \"none_policy\"},\n"
            "  \"sampling_profile\": {\"enabled\": true, \"policy\": \"none\", \"mode\": \"%s\", \"stochastic_samples\": 0, "
            "\"top_p_evaluations\": 0, \"beam_width\": 1, \"disabled_reason\": \"none_policy\"},\n"
            "  \"long_context_profile\": {\"enabled\": true, \"policy\": \"%s\", \"target_ctx_tokens\": %u, \"rss_limit_bytes\": 0, "
            "\"kv_quality_checks\": 0, \"soak_seconds\": 0, \"disabled_reason\": %s},\n",
            scratch_policy, (unsigned long long)qxg_device_bytes(ctx), dequant_profile ? "true" : "false", kernel_policy,
            (unsigned long long)(final_head ? decode_tokens : 0), (unsigned long long)(final_head ? (uint64_t)decode_tokens * vocab * 8 : 0),
            thread_policy, threads, threads, (unsigned long long)((uint64_t)steps * (layers - start_layer)),
            (unsigned long long)((uint64_t)steps * (layers - start_layer)), pool ? "" : ", \"disabled_reason\": \"serial_policy\"",
            simd_policy, avx2 ? "" : ", \"disabled_reason\": \"scalar_policy\"", (unsigned long long)qxg_device_bytes(ctx),
            t_load, temperature > 0.0 ? "temperature_top_k" : "greedy", long_context_policy, ctx4k ? 4096u : 0u,
            ctx4k ? "null" : "\"none_policy\"");
    const char *note = replay ? "hybrid one-token replay from an injected F32 residual through the requested layer suffix"
        : final_head ? (steps > 1 ? (prompt_count > 1
              ? "tokenized Qwen3 prompt prefill followed by greedy generation: fixed prompt IDs and selected tokens are embedded at their positions with persistent per-layer INT8 KV; the complete Q6_K head runs only for generation outputs"
              : "greedy multi-token Qwen3 forward: every selected token is re-embedded, position and per-layer INT8 KV advance, then all 48 layers, final RMSNorm, and the complete Q6_K vocabulary head run again")
              : "one-token Qwen3 forward through 48 layers, final RMSNorm, and complete Q6_K vocabulary head; tokenizer parity and multi-token execution are separate gates")
        : "one-token Qwen3 transformer forward with real attention, dynamic INT8 KV, and top-8 MoE; final head disabled";
    fprintf(out, "  \"note\": \"%s\"\n}\n", note);
done:
#undef FAIL
    free(s_lay); free(s_att); free(s_moe); free(s_ks); free(s_vs); free(s_ws); free(s_rw); free(s_ids); free(s_k); free(s_v);
    free(s_norm); free(s_lg); free(s_tid); free(s_tl); free(s_tok); free(s_ms);
    probe_scan_free(&ps);
    free(logits);
    free(generated);
    if (ctx) qxg_close(ctx);
    qxf_close(&f);
    return ok;
}

/* reference qx_dump_state_loop_probe_summary (src/qx_format.c:6721-6733): one prompt token,
 * `steps` forward steps, the default policies */
int qx_dump_state_loop_probe_summary(const char *path, const char *tokens_path, uint32_t prompt_token, uint32_t steps,
        uint32_t layers, uint32_t ctx_tokens, const char *kv_format, const char *activation_format, int real_kv,
        int projection_matvec, int residual_vector, int residual_carry, int numeric_deltas, int delta_vectors,
        int attention_output_vector, int causal_attention, int rope_gqa_attention, int full_moe, int final_head, int bench,
        uint32_t residual_dims, const char *norm_name, uint32_t top_k, uint32_t scan, uint32_t logits_top_n,
        double temperature, uint32_t seed, const char *residual_dump_dir, uint32_t start_layer,
        const char *residual_input_path, const char *kv_snapshot_out_path, const char *kv_snapshot_in_path, FILE *out,
        char *err, uint64_t err_len) {
    if (final_head && (steps == 0 || steps > 64)) {
        qxh_set_err(err, err_len, "--final-head requires --full-moe, 1..64 steps, all manifest layers, and temperature 0");
        return 0;
    }
    if (steps == 0) steps = 1;
    if (steps > 64) steps = 64;
    return qx_dump_prompt_state_loop_probe_summary(path, tokens_path, &prompt_token, 1, steps, layers, ctx_tokens, kv_format,
        activation_format, "ephemeral", "baseline", "serial", 1, "scalar", "none", "none", "none", "none", "none", "none",
        "none", 0, real_kv, projection_matvec, residual_vector, residual_carry, numeric_deltas, delta_vectors,
        attention_output_vector, causal_attention, rope_gqa_attention, full_moe, final_head, bench, residual_dims, norm_name,
        top_k, scan, logits_top_n, temperature, seed, residual_dump_dir, start_layer, residual_input_path,
        kv_snapshot_out_path, kv_snapshot_in_path, out, err, err_len);
}
