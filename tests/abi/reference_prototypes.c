/* ABI check of the drop-in boundary: the reference's declarations of the probe entry points
 * this build replaces (reference include/qx_format.h:140, 156-158, 161-163, verbatim), in
 * one translation unit with this build's include/qx_host.h.  A prototype that differs fails
 * to compile (conflicting types); a missing export fails to link against libqxhost.so.  The
 * program only takes each function's address: it runs nothing on a device. */
#include <stdint.h>
#include <stdio.h>

#include "qx_host.h"

int qx_dump_decode_block_summary(const char *path, const char *name, uint64_t block_index, FILE *out, char *err, uint64_t err_len);
int qx_dump_q8_k_activation_probe_summary(uint32_t values, const char *inject, FILE *out, char *err, uint64_t err_len);
int qx_dump_state_loop_probe_summary(const char *path, const char *tokens_path, uint32_t prompt_token, uint32_t steps, uint32_t layers, uint32_t ctx_tokens, const char *kv_format, const char *activation_format, int real_kv, int projection_matvec, int residual_vector, int residual_carry, int numeric_deltas, int delta_vectors, int attention_output_vector, int causal_attention, int rope_gqa_attention, int full_moe, int final_head, int bench, uint32_t residual_dims, const char *norm_name, uint32_t top_k, uint32_t scan, uint32_t logits_top_n, double temperature, uint32_t seed, const char *residual_dump_dir, uint32_t start_layer, const char *residual_input_path, const char *kv_snapshot_out_path, const char *kv_snapshot_in_path, FILE *out, char *err, uint64_t err_len);
int qx_dump_prompt_state_loop_probe_summary(const char *path, const char *tokens_path, const uint32_t *prompt_tokens, uint32_t prompt_count, uint32_t generation_steps, uint32_t layers, uint32_t ctx_tokens, const char *kv_format, const char *activation_format, const char *scratch_policy, const char *kernel_policy, const char *thread_policy, uint32_t threads, const char *simd_policy, const char *expert_cache_policy, const char *cuda_policy, const char *prefill_gemm_policy, const char *speculative_policy, const char *kv2_policy, const char *sampling_policy, const char *long_context_policy, int dequant_profile, int real_kv, int projection_matvec, int residual_vector, int residual_carry, int numeric_deltas, int delta_vectors, int attention_output_vector, int causal_attention, int rope_gqa_attention, int full_moe, int final_head, int bench, uint32_t residual_dims, const char *norm_name, uint32_t top_k, uint32_t scan, uint32_t logits_top_n, double temperature, uint32_t seed, const char *residual_dump_dir, uint32_t start_layer, const char *residual_input_path, const char *kv_snapshot_out_path, const char *kv_snapshot_in_path, FILE *out, char *err, uint64_t err_len);
int qx_dump_attention_stage_probe_summary(const char *path, uint32_t layer, const char *layer_input_path, const char *output_dir, const char *activation_mode, const char *kv_format, FILE *out, char *err, uint64_t err_len);
int qx_dump_moe_stage_probe_summary(const char *path, uint32_t layer, const char *ffn_input_path, const char *output_dir, const char *activation_mode, FILE *out, char *err, uint64_t err_len);
int qx_dump_final_head_probe_summary(const char *path, const char *residual_path, const char *output_dir, const char *activation_mode, uint32_t top_n, FILE *out, char *err, uint64_t err_len);

int main(void) {
    void *const entry[] = {
        (void *)qx_dump_decode_block_summary,
        (void *)qx_dump_q8_k_activation_probe_summary,
        (void *)qx_dump_state_loop_probe_summary,
        (void *)qx_dump_prompt_state_loop_probe_summary,
        (void *)qx_dump_attention_stage_probe_summary,
        (void *)qx_dump_moe_stage_probe_summary,
        (void *)qx_dump_final_head_probe_summary,
    };
    unsigned n = 0;
    for (unsigned i = 0; i < sizeof(entry) / sizeof(entry[0]); ++i) n += entry[i] != NULL;
    printf("%u\n", n);
    return n == sizeof(entry) / sizeof(entry[0]) ? 0 : 1;
}
