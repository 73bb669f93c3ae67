/* qxqxf — CLI for the GPU path with the reference's sub-command names and flags
 * for the probes on the decode path (reference src/qx_qxf_main.c:235-258,
 * 1219-1237, 1671-1697, 1726-1809).  Exit codes: 0 ok, 1 runtime failure, 2 usage. */
#include "qx_host.h"

#include <errno.h>
#include <stdlib.h>
#include <string.h>

static void usage(const char *argv0) {
    fprintf(stderr,
            "usage:\n"
            "  %s decode-block --in FILE --name TENSOR --block N\n"
            "  %s final-head-probe --in FILE --residual R.f32 --out-dir DIR [--activation f32|q8_k_compat] [--top-n N]\n"
            "  %s state-loop-probe --in FILE --prompt-token T[,T...] --steps N --ctx C --kv int8 --full-moe\n"
            "        [--final-head] [--top-n N] [--dump-residuals DIR] [--bench] [--activation f32|q8_k_compat]\n"
            "  %s q8-k-activation-probe --values N [--inject none|zero|nan|inf|positive|negative|edge]\n"
            "  %s generate-model --out FILE [--layers L] [--vocab V] [--experts E] [--seed S] [--no-embedding] [--no-head] [--mix]\n",
            argv0, argv0, argv0, argv0, argv0);
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
        const char *in = NULL, *kv = "int8", *act = "f32", *dump = NULL;
        uint32_t prompt[64], n_prompt = 0, steps = 1, ctx = 64, top_n = 5;
        int full_moe = 0, final_head = 0, bench = 0;
        for (int i = 2; i < argc; ++i) {
            if (!strcmp(argv[i], "--in") && i + 1 < argc) in = argv[++i];
            else if (!strcmp(argv[i], "--prompt-token") && i + 1 < argc) {
                char *s = argv[++i];
                for (char *tok = strtok(s, ","); tok; tok = strtok(NULL, ",")) {
                    if (n_prompt >= 64 || !parse_u32(tok, &prompt[n_prompt])) { usage(argv[0]); return 2; }
                    ++n_prompt;
                }
            }
            else if (!strcmp(argv[i], "--steps") && i + 1 < argc) { if (!parse_u32(argv[++i], &steps)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--ctx") && i + 1 < argc) { if (!parse_u32(argv[++i], &ctx)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--top-n") && i + 1 < argc) { if (!parse_u32(argv[++i], &top_n)) { usage(argv[0]); return 2; } }
            else if (!strcmp(argv[i], "--kv") && i + 1 < argc) kv = argv[++i];
            else if (!strcmp(argv[i], "--activation") && i + 1 < argc) act = argv[++i];
            else if (!strcmp(argv[i], "--dump-residuals") && i + 1 < argc) dump = argv[++i];
            else if (!strcmp(argv[i], "--full-moe")) full_moe = 1;
            else if (!strcmp(argv[i], "--final-head")) final_head = 1;
            else if (!strcmp(argv[i], "--bench")) bench = 1;
            else { usage(argv[0]); return 2; }
        }
        if (!in || !n_prompt) { usage(argv[0]); return 2; }
        if (!full_moe) { fprintf(stderr, "state-loop-probe failed: the GPU path implements --full-moe only\n"); return 1; }
        /* --steps counts forward steps as in the reference (prompt + generation - 1) */
        if (steps < n_prompt) { fprintf(stderr, "state-loop-probe failed: --steps must cover the prompt\n"); return 1; }
        const uint32_t gen = steps - n_prompt + 1;
        if (!qx_dump_prompt_state_loop_gpu(in, prompt, n_prompt, gen, ctx, kv, act, final_head, top_n, dump, bench, stdout, err, sizeof(err))) {
            fprintf(stderr, "state-loop-probe failed: %s\n", err);
            return 1;
        }
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
        if (!qx_dump_q8_k_activation_probe_gpu(values, inject, stdout, err, sizeof(err))) {
            fprintf(stderr, "q8-k-activation-probe failed: %s\n", err);
            return 1;
        }
        return 0;
    }
    if (!strcmp(cmd, "generate-model")) {
        const char *outp = NULL;
        qxgen_spec sp = {48, 151936, 128, 1, 1, 1, 0, 0};
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
