/* qxqxf — CLI of the GPU path with the reference's sub-command names, flags and defaults
 * for the probes on the decode path (reference src/qx_qxf_main.c: state-loop-probe
 * 1726-1809, prompt-state-loop-probe 395-563, attention-stage-probe 1641-1669,
 * moe-stage-probe 1613-1639, final-head-probe 1671-1697, decode-block 235-258,
 * q8-k-activation-probe 1219-1237).  prompt-state-loop-probe takes the prompt as token
 * ids (--prompt-ids), the tokenizer being outside this build.  Exit codes: 0 ok,
 * 1 runtime failure, 2 usage. */
#include "qx_host.h"

#include <errno.h>
#include <stdlib.h>
#include <string.h>

static void usage(const char *argv0) {
    fprintf(stderr,
            "usage:\n"
            "  %s decode-block --in FILE --name TENSOR --block N\n"
            "  %s final-head-probe --in FILE --residual R.f32 --out-dir DIR [--activation f32|q8_k_compat] [--top-n N]\n"
            "  %s state-loop-probe --in FILE [--tokens T.tsv] --prompt-token T --steps N --layers L --ctx C --kv int8\n"
            "        --activation f32|q8_k_compat --temperature 0 --seed S --full-moe [--start-layer N --residual-in R.f32]\n"
            "        [--final-head --top-n N] [--dump-residuals DIR] [--kv-snapshot-out F | --kv-snapshot-in F] [--bench]\n"
            "        [--top-k K] [--scan S]\n"
            "  %s prompt-state-loop-probe --in FILE --prompt-ids A,B,... --generate N --layers 48 --ctx 16 --kv int8\n"
            "        --activation f32|q8_k_compat --full-moe --final-head [--scratch-policy P --kernel-policy P\n"
            "        --thread-policy serial|pool --threads N --simd-policy P ...] [--bench] [--top-n N] [--kv-snapshot-out F]\n"
            "  %s attention-stage-probe --in FILE --layer L --layer-in X.f32 --out-dir DIR [--activation A] [--kv f32|f16]\n"
            "  %s moe-stage-probe --in FILE --layer L --ffn-inp X.f32 --out-dir DIR [--activation A]\n"
            "  %s q8-k-activation-probe --values N [--inject none|zero|nan|inf|positive|negative|edge]\n"
            "  %s generate-model --out FILE [--layers L] [--vocab V] [--experts E] [--seed S] [--no-embedding] [--no-head] [--mix]\n",
            argv0, argv0, argv0, argv0, argv0, argv0, argv0, argv0);
}

static int parse_u32(const char *s, uint32_t *out) {
    char *end = NULL;
    errno = 0;
    unsigned long v = strtoul(s, &end, 10);
    if (errno || !end || *end || v > 0xfffffffful) return 0;
    *out = (uint32_t)v;
    return 1;
}

int main(int argc, char **argv) {
    if (argc < 2) { usage(argv[0]); return 2; }
    char err[512] = {0};
    const char *cmd = argv[1];
    if (!strcmp(cmd, "decode-block")) {
        const char *in = NULL, *name = NULL;
        uint64_t block = 0;
        for (int i = 2; i < argc; ++i) {
            if (!strcmp(argv[i], "--in") && i + 1 < argc) in = argv[++i];
            else if (!strcmp(argv[i], "--name") && i + 1 < argc) name = argv[++i];
            else if (!strcmp(argv[i], "--block") && i + 1 < argc) block = strtoull(argv[++i], NULL, 10);
            else { usage(argv[0]); return 2; }
        }
        if (!in || !name) { usage(argv[0]); return 2; }
        if (!qx_dump_decode_block_summary(in, name, block, stdout, err, sizeof(err))) { fprintf(stderr, "decode-block failed: %s\n", err); return 1; }
        return 0;
    }
    if (!strcmp(cmd, "final-head-probe")) {
        const char *in = NULL, *res = NULL, *dir = NULL, *act = "f32";
        uint32_t top_n = 5;
        for (int i = 2; i < argc; ++i) {
            if (!strcmp(argv[i], "--in") && i + 1 < argc) in = argv[++i];
            else if (!strcmp(argv[i], "--residual") && i + 1 < argc) res = argv[++i];
            else if (!strcmp(argv[i], "--out-dir") && i + 1 < argc) dir = argv[++i];
            else if (!strcmp(argv[i], "--activation") && i + 1 < argc) act = argv[++i];
            else if (!strcmp(argv[i], "--top-n") && i + 1 < argc) {
                if (!parse_u32(argv[++i], &top_n) || top_n == 0 || top_n > 32) { usage(argv[0]); return 2; }
            } else { usage(argv[0]); return 2; }
        }
        if (!in || !res || !dir) { usage(argv[0]); return 2; }
        if (!qx_dump_final_head_probe_summary(in, res, dir, act, top_n, stdout, err, sizeof(err))) { fprintf(stderr, "final-head-probe failed: %s\n", err); return 1; }
        return 0;
    }
    if (!strcmp(cmd, "state-loop-probe")) {
        /* defaults and flag implications of the reference (src/qx_qxf_main.c:1726-1790) */
        const char *in = NULL, *tokens = NULL, *kv = "int8", *act = "f32", *dump = NULL, *res_in = NULL;
        const char *snap_out = NULL, *snap_in = NULL, *norm = NULL;
        int real_kv = 0, pmv = 0, rvec = 0, rcarry = 0, ndelta = 0, dvec = 0, aov = 0, causal = 0, rope = 0, full_moe = 0;
        int final_head = 0, bench = 0, start_set = 0;
        uint32_t start_layer = 0, residual_dims = 64, prompt = 0, steps = 1, layers = 1, ctx = 16, top_k = 5, scan = 64;
        uint32_t top_n = 5, seed = 1;
        double temperature = 0.0;
        for (int i = 2; i < argc; ++i) {
            const char *a = argv[i];
            const int more = i + 1 < argc;
            if (!strcmp(a, "--in") && more) in = argv[++i];
            else if (!strcmp(a, "--tokens") && more) tokens = argv[++i];
            else if (!strcmp(a, "--prompt-token") && more) prompt = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--steps") && more) steps = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--layers") && more) layers = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--ctx") && more) ctx = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--kv") && more) kv = argv[++i];
            else if (!strcmp(a, "--activation") && more) act = argv[++i];
            else if (!strcmp(a, "--real-kv")) real_kv = 1;
            else if (!strcmp(a, "--projection-matvec")) { pmv = real_kv = 1; }
            else if (!strcmp(a, "--residual-vector")) { rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--residual-carry")) { rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--numeric-deltas")) { ndelta = rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--delta-vectors")) { dvec = ndelta = rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--attention-output-vector")) { aov = dvec = ndelta = rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--causal-attention")) { causal = aov = dvec = ndelta = rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--rope-gqa-attention")) { rope = causal = aov = dvec = ndelta = rcarry = rvec = pmv = real_kv = 1; }
            else if (!strcmp(a, "--full-moe")) {
                full_moe = rope = causal = aov = dvec = ndelta = rcarry = rvec = pmv = real_kv = 1;
                residual_dims = 2048;
            }
            else if (!strcmp(a, "--final-head")) final_head = 1;
            else if (!strcmp(a, "--bench")) bench = 1;
            else if (!strcmp(a, "--dump-residuals") && more) dump = argv[++i];
            else if (!strcmp(a, "--residual-in") && more) res_in = argv[++i];
            else if (!strcmp(a, "--kv-snapshot-out") && more) snap_out = argv[++i];
            else if (!strcmp(a, "--kv-snapshot-in") && more) snap_in = argv[++i];
            else if (!strcmp(a, "--start-layer") && more) {
                if (!parse_u32(argv[++i], &start_layer)) { usage(argv[0]); return 2; }
                start_set = 1;
            }
            else if (!strcmp(a, "--residual-dims") && more) residual_dims = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--norm") && more) norm = argv[++i];
            else if (!strcmp(a, "--top-k") && more) top_k = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--scan") && more) scan = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--top-n") && more) top_n = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--temperature") && more) temperature = strtod(argv[++i], NULL);
            else if (!strcmp(a, "--seed") && more) seed = (uint32_t)strtoul(argv[++i], NULL, 10);
            else { usage(argv[0]); return 2; }
        }
        if (!in || start_set != (res_in != NULL) || (snap_out && snap_in)) { usage(argv[0]); return 2; }
        if (!qx_dump_state_loop_probe_summary(in, tokens, prompt, steps, layers, ctx, kv, act, real_kv, pmv, rvec, rcarry,
                                              ndelta, dvec, aov, causal, rope, full_moe, final_head, bench, residual_dims, norm,
                                              top_k, scan, top_n, temperature, seed, dump, start_layer, res_in, snap_out,
                                              snap_in, stdout, err, sizeof(err))) {
            fprintf(stderr, "state-loop-probe failed: %s\n", err);
            return 1;
        }
        return 0;
    }
    if (!strcmp(cmd, "prompt-state-loop-probe")) {
        /* defaults of the reference (src/qx_qxf_main.c:395-420) */
        const char *in = NULL, *kv = "int8", *act = "f32", *scratch = "ephemeral", *kernel = "baseline";
        const char *thread = "serial", *simd = "scalar", *ecache = "none", *cuda = "none", *pgemm = "none";
        const char *spec = "none", *kv2 = "none", *sampling = "none", *longctx = "none", *snap_out = NULL;
        uint32_t ids[64], count = 0, gen = 0, layers = 48, ctx = 16, top_n = 5, seed = 7, threads = 1;
        double temperature = 0.0;
        int full_moe = 0, final_head = 0, bench = 0, dq = 0;
        for (int i = 2; i < argc; ++i) {
            const char *a = argv[i];
            const int more = i + 1 < argc;
            if (!strcmp(a, "--in") && more) in = argv[++i];
            else if (!strcmp(a, "--prompt-ids") && more) {
                char *s = argv[++i];
                for (char *t = strtok(s, ","); t; t = strtok(NULL, ",")) {
                    if (count >= 64 || !parse_u32(t, &ids[count])) { usage(argv[0]); return 2; }
                    ++count;
                }
            }
            else if ((!strcmp(a, "--tokenizer") || !strcmp(a, "--text-file")) && more) {
                fprintf(stderr, "prompt-state-loop-probe failed: the tokenizer is not part of this build; pass --prompt-ids\n");
                return 2;
            }
            else if (!strcmp(a, "--generate") && more) gen = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--layers") && more) layers = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--ctx") && more) ctx = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--kv") && more) kv = argv[++i];
            else if (!strcmp(a, "--activation") && more) act = argv[++i];
            else if (!strcmp(a, "--io-backend") && more) ++i;   /* the file is always memory-mapped here */
            else if (!strcmp(a, "--scratch-policy") && more) scratch = argv[++i];
            else if (!strcmp(a, "--kernel-policy") && more) kernel = argv[++i];
            else if (!strcmp(a, "--thread-policy") && more) thread = argv[++i];
            else if (!strcmp(a, "--simd-policy") && more) simd = argv[++i];
            else if (!strcmp(a, "--expert-cache-policy") && more) ecache = argv[++i];
            else if (!strcmp(a, "--cuda-policy") && more) cuda = argv[++i];
            else if (!strcmp(a, "--prefill-gemm-policy") && more) pgemm = argv[++i];
            else if (!strcmp(a, "--speculative-policy") && more) spec = argv[++i];
            else if (!strcmp(a, "--kv2-policy") && more) kv2 = argv[++i];
            else if (!strcmp(a, "--sampling-policy") && more) sampling = argv[++i];
            else if (!strcmp(a, "--long-context-policy") && more) longctx = argv[++i];
            else if (!strcmp(a, "--threads") && more) {
                if (!parse_u32(argv[++i], &threads)) { fprintf(stderr, "prompt-state-loop-probe failed: invalid --threads\n"); return 2; }
            }
            else if (!strcmp(a, "--temperature") && more) temperature = strtod(argv[++i], NULL);
            else if (!strcmp(a, "--seed") && more) seed = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--top-n") && more) top_n = (uint32_t)strtoul(argv[++i], NULL, 10);
            else if (!strcmp(a, "--kv-snapshot-out") && more) snap_out = argv[++i];
            else if (!strcmp(a, "--parse-special")) {}
            else if (!strcmp(a, "--full-moe")) full_moe = 1;
            else if (!strcmp(a, "--final-head")) final_head = 1;
            else if (!strcmp(a, "--bench")) bench = 1;
            else if (!strcmp(a, "--dequant-profile")) dq = 1;
            else { usage(argv[0]); return 2; }
        }
        if (!in || !count || !full_moe || !final_head) { usage(argv[0]); return 2; }
        if (!qx_dump_prompt_state_loop_probe_summary(in, NULL, ids, count, gen, layers, ctx, kv, act, scratch, kernel, thread,
                                                     threads, simd, ecache, cuda, pgemm, spec, kv2, sampling, longctx, dq, 1,
                                                     1, 1, 1, 1, 1, 1, 1, 1, full_moe, final_head, bench, 2048u, NULL, 8u,
                                                     151936u, top_n, temperature, seed, NULL, 0u, NULL, snap_out, NULL,
                                                     stdout, err, sizeof(err))) {
            fprintf(stderr, "prompt-state-loop-probe failed: %s\n", err);
            return 1;
        }
        return 0;
    }
    if (!strcmp(cmd, "attention-stage-probe") || !strcmp(cmd, "moe-stage-probe")) {
        const int attn = !strcmp(cmd, "attention-stage-probe");
        const char *in = NULL, *x = NULL, *dir = NULL, *act = "f32", *kv = "f32";
        uint32_t layer = 0;
        for (int i = 2; i < argc; ++i) {
            const char *a = argv[i];
            const int more = i + 1 < argc;
            if (!strcmp(a, "--in") && more) in = argv[++i];
            else if (attn && !strcmp(a, "--layer-in") && more) x = argv[++i];
            else if (!attn && !strcmp(a, "--ffn-inp") && more) x = argv[++i];
            else if (!strcmp(a, "--out-dir") && more) dir = argv[++i];
            else if (!strcmp(a, "--activation") && more) act = argv[++i];
            else if (attn && !strcmp(a, "--kv") && more) kv = argv[++i];
            else if (!strcmp(a, "--layer") && more) {
                if (!parse_u32(argv[++i], &layer)) { usage(argv[0]); return 2; }
            } else { usage(argv[0]); return 2; }
        }
        if (!in || !x || !dir) { usage(argv[0]); return 2; }
        const int ok = attn ? qx_dump_attention_stage_probe_summary(in, layer, x, dir, act, kv, stdout, err, sizeof(err))
                            : qx_dump_moe_stage_probe_summary(in, layer, x, dir, act, stdout, err, sizeof(err));
        if (!ok) { fprintf(stderr, "%s failed: %s\n", cmd, err); return 1; }
        return 0;
    }
    if (!strcmp(cmd, "q8-k-activation-probe")) {
        const char *inject = "none";
        uint32_t values = 0;
        int seen = 0;
        for (int i = 2; i < argc; ++i) {
            if (!strcmp(argv[i], "--values") && i + 1 < argc) {
                if (!parse_u32(argv[++i], &values)) { fprintf(stderr, "q8-k-activation-probe failed: invalid --values\n"); return 2; }
                seen = 1;
            } else if (!strcmp(argv[i], "--inject") && i + 1 < argc) inject = argv[++i];
            else { usage(argv[0]); return 2; }
        }
        if (!seen) { fprintf(stderr, "q8-k-activation-probe failed: invalid --values\n"); return 2; }
        if (!qx_dump_q8_k_activation_probe_summary(values, inject, stdout, err, sizeof(err))) {
            fprintf(stderr, "q8-k-activation-probe failed: %s\n", err);
            return 1;
        }
        return 0;
    }
    if (!strcmp(cmd, "generate-model")) {
        const char *outp = NULL;
        qxgen_spec sp = {48, 151936, 128, 1, 1, 1, 0, 0, 0};
        uint32_t seed = 1;
        for (int i = 2; i < argc; ++i) {
            if (!strcmp(argv[i], "--out") && i + 1 < argc) outp = argv[++i];
            else if (!strcmp(argv[i], "--layers") && i + 1 < argc) { if (!parse_u32(argv[++i], &sp.layers)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--vocab") && i + 1 < argc) { if (!parse_u32(argv[++i], &sp.vocab)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--experts") && i + 1 < argc) { if (!parse_u32(argv[++i], &sp.experts)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--seed") && i + 1 < argc) { if (!parse_u32(argv[++i], &seed)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--no-embedding")) sp.with_embedding = 0;
            else if (!strcmp(argv[i], "--no-head")) sp.with_head = 0;
            else if (!strcmp(argv[i], "--mix")) sp.mix = 1;
            else { usage(argv[0]); return 2; }
        }
        if (!outp) { usage(argv[0]); return 2; }
        sp.seed = seed;
        uint64_t size = 0;
        if (!qxgen_write(outp, &sp, &size, err, sizeof(err))) { fprintf(stderr, "generate-model failed: %s\n", err); return 1; }
        printf("{\"out\": \"%s\", \"file_size\": %llu}\n", outp, (unsigned long long)size);
        return 0;
    }
    usage(argv[0]);
    return 2;
}
