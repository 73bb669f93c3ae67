/* Host-side C API of the MI355X build: QXF1 tensor file access, the seeded
 * synthetic-model writer, and the probes/state loop that drive the GPU.
 *
 * Conventions follow the reference C API (include/qx_format.h:104-172 of the
 * reference): functions return 1 on success and 0 on failure, and write a
 * message into the caller's (char *err, uint64_t err_len) buffer.  JSON goes to a
 * caller FILE*.  The structs below are the on-disk QXF1 layout
 * (reference include/qx_format.h:12-82), byte for byte: a 272-byte header and
 * 208-byte directory entries, little-endian, every offset 4096-aligned.
 */
#ifndef QX_HOST_H
#define QX_HOST_H

#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QXF_MAGIC "QXF1"
#define QXF_VERSION 1u
#define QXF_NAME_MAX 96u
#define QXF_MAX_DIMS 4u
#define QXF_ALIGN 4096ull

/* ggml type ids stored in qxf_dir_entry.flags */
enum { QXT_F32 = 0, QXT_Q4_K = 12, QXT_Q5_K = 13, QXT_Q6_K = 14, QXT_IQ2_XS = 17,
       QXT_IQ3_XXS = 18, QXT_IQ3_S = 21, QXT_IQ2_S = 22, QXT_IQ4_XS = 23 };

typedef struct qxf_manifest {
    uint32_t model_type;          /* 1 dense, 2 MoE */
    uint32_t quant_type;          /* 1..5 */
    uint32_t layers, hidden, intermediate, q_heads, kv_heads, head_dim, vocab, max_ctx;
    uint32_t experts, experts_per_token, moe_intermediate;
} qxf_manifest;

typedef struct qxf_header {
    char magic[4];
    uint32_t version, header_size, dir_entry_size, tensor_count;
    uint64_t dir_offset, data_offset, file_size, manifest_checksum;
    qxf_manifest manifest;
    uint8_t reserved[160];
} qxf_header;

typedef struct qxf_dir_entry {
    char name[QXF_NAME_MAX];
    uint32_t dtype, quant, rank;
    uint64_t dims[QXF_MAX_DIMS];  /* dims[0] = contiguous input dim, dims[1] = rows, dims[2] = experts */
    uint64_t offset, byte_size;
    uint32_t group_size;
    uint32_t flags;               /* ggml type */
    uint64_t checksum;            /* FNV-1a-64 of the tensor bytes */
    uint8_t reserved[32];
} qxf_dir_entry;

typedef struct qxf_file {
    int fd;
    qxf_header header;
    qxf_dir_entry *dir;
    const uint8_t *map;           /* whole file, PROT_READ / MAP_PRIVATE */
} qxf_file;

uint64_t qxf_fnv1a64(const void *data, uint64_t len);
uint64_t qxf_fnv1a64_update(uint64_t h, const void *data, uint64_t len);
/* Bytes per 256-value block (or 4 for F32 with 1-value blocks); 0 if unsupported. */
int qxf_type_block(uint32_t ggml_type, uint64_t *block_values, uint64_t *block_bytes);

/* Open + validate (header, manifest FNV, exact size, alignment, names, traits,
 * dims, byte sizes, duplicates, overlaps), then mmap.  reference qx_open_file,
 * src/qx_format.c:712-841. */
int qxf_open(const char *path, qxf_file *out, char *err, uint64_t err_len);
void qxf_close(qxf_file *f);
const qxf_dir_entry *qxf_find(const qxf_file *f, const char *name);
const uint8_t *qxf_data(const qxf_file *f, const qxf_dir_entry *t);
/* reference qx_verify_tensor_checksum, src/qx_format.c:903-943 */
int qxf_verify(const qxf_file *f, const qxf_dir_entry *t, char *err, uint64_t err_len);

/* ---- seeded synthetic model writer (the configs' random-init model) ---- */
typedef struct qxgen_spec {
    uint32_t layers;        /* 0..48; manifest.layers is always this value */
    uint32_t vocab;         /* 151936 for the full model */
    uint32_t experts;       /* 8..128 */
    uint32_t with_embedding;/* token_embd.weight (Q4_K) */
    uint32_t with_head;     /* output_norm.weight + output.weight (Q6_K) */
    uint64_t seed;
    uint32_t threads;       /* 0 = all online CPUs (capped at 16) */
    uint32_t mix;           /* 0: IQ4_XS attention, IQ2_XS gate/up, IQ3_XXS down in every layer;
                               1: the real checkpoint's per-layer mix, layer l by l % 4:
                               0 -> (IQ4_XS v/o, IQ2_XS gate/up, IQ3_XXS down), 1 -> (Q5_K, IQ2_S, IQ4_XS),
                               2 -> (IQ4_XS, IQ2_XS, IQ3_S), 3 -> (Q5_K, IQ2_S, IQ3_S); q/k stay IQ4_XS */
    uint32_t outliers;      /* planted outlier channels (a test input, not a model distribution).
                               0: none.  1: single x1000 channels - channel 128 k + 5 of every
                               2048-long norm and channel 5 of the q/k norms, fp16 d x1000 in V row
                               128 k + 3 (the context) and O row 11 (the residual stream).  2: a
                               compound stress pattern - as 1, plus x1e6 in channel 1001 of the
                               attention and output norms and fp16 d x1000 in gate row 7 and down
                               row 13 of every expert (h groups spanning ~1e4-1e5, and expert
                               outputs that cancel in channel 13).  3: exponent-31 fp16 block
                               scales (+inf, -inf, NaN, -NaN by block, which the reference reads
                               as +-65504) in every block of Q row 100, K row 7, V row 3, O row 11
                               and gate row 7, up row 9, down row 13 of every expert; no norm
                               outliers */
} qxgen_spec;

/* Writes a QXF1 file at `path` (truncating).  The bytes are a pure function of
 * (spec minus threads).  Block distributions: per-format ranges documented in
 * qxgen.c.  Returns total file size in *file_size. */
int qxgen_write(const char *path, const qxgen_spec *spec, uint64_t *file_size, char *err, uint64_t err_len);
/* Same, into an anonymous in-memory file; *path_out receives "/proc/self/fd/N".
 * The descriptor stays open for the life of the process unless closed by
 * qxgen_memfd_close(fd). */
int qxgen_memfd(const qxgen_spec *spec, char *path_out, uint64_t path_len, int *fd_out, char *err, uint64_t err_len);
void qxgen_memfd_close(int fd);

/* ---- GPU-backed probes with the reference's entry-point semantics ---- */
struct qxg_ctx;

typedef struct qx_gpu_model_info {
    uint32_t layers, vocab, experts;
    int has_embedding, has_head;
    uint64_t tensor_bytes;      /* sum of uploaded tensor bytes */
    uint32_t tensors;
} qx_gpu_model_info;

/* Opens a QXF1 file (qxf_open), optionally verifies every tensor's FNV-1a-64
 * (the reference verifies the head's on every token, src/qx_format.c:3631-3632;
 * here it is done once, at load), uploads every tensor with qxg_upload_tensor and
 * binds layers [0, manifest.layers).  Files without token_embd / output tensors
 * bind without them. */
int qx_gpu_load(struct qxg_ctx *ctx, const char *path, int verify_checksums, qx_gpu_model_info *info,
                char *err, uint64_t err_len);

/* reference qx_dump_decode_block_summary (include/qx_format.h:140): decodes one
 * 256-value block of tensor `name` on the GPU and prints its FNV over the floats. */
int qx_dump_decode_block_summary(const char *path, const char *name, uint64_t block_index, FILE *out, char *err, uint64_t err_len);
/* reference qx_dump_final_head_probe_summary (include/qx_format.h:163). */
int qx_dump_final_head_probe_summary(const char *path, const char *residual_path, const char *output_dir,
        const char *activation_mode, uint32_t top_n, FILE *out, char *err, uint64_t err_len);
/* reference qx_dump_q8_k_activation_probe_summary (include/qx_format.h:156), same name
 * and prototype: the probe's fixed inputs (inject: none, zero, nan, inf, positive,
 * negative, edge) quantized to Q8_K blocks on the GPU; the reference's JSON keys, block
 * bytes and error messages. */
int qx_dump_q8_k_activation_probe_summary(uint32_t values, const char *inject, FILE *out, char *err, uint64_t err_len);
/* reference qx_dump_state_loop_probe_summary and qx_dump_prompt_state_loop_probe_summary
 * (include/qx_format.h:157-158), same prototypes: the state loop of
 * src/qx_format.c:5970-6733 on the GPU.  The reference's argument checks run first, with
 * its messages; the device path then requires --full-moe (full_moe, rope_gqa_attention and
 * causal_attention set) and INT8 KV, and rejects the probe-level skeleton modes with an
 * error.  Supported: prompt prefill then generation (1..64 steps), --layers below the
 * manifest's, --start-layer/--residual-in replay, --kv-snapshot-out/--kv-snapshot-in
 * (QXKVSNP1; the continuation token must be the snapshot's next token), --dump-residuals,
 * --final-head (greedy, the device head) or, without it, the reference's token scan and
 * sampler, --bench, f32 and q8_k_compat activations.  The JSON carries the reference's
 * keys; thread/simd policies are validated and reported (the device ignores them). */
int qx_dump_state_loop_probe_summary(const char *path, const char *tokens_path, uint32_t prompt_token, uint32_t steps,
        uint32_t layers, uint32_t ctx_tokens, const char *kv_format, const char *activation_format, int real_kv,
        int projection_matvec, int residual_vector, int residual_carry, int numeric_deltas, int delta_vectors,
        int attention_output_vector, int causal_attention, int rope_gqa_attention, int full_moe, int final_head, int bench,
        uint32_t residual_dims, const char *norm_name, uint32_t top_k, uint32_t scan, uint32_t logits_top_n,
        double temperature, uint32_t seed, const char *residual_dump_dir, uint32_t start_layer,
        const char *residual_input_path, const char *kv_snapshot_out_path, const char *kv_snapshot_in_path, FILE *out,
        char *err, uint64_t err_len);
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
        char *err, uint64_t err_len);
/* reference qx_dump_attention_stage_probe_summary and qx_dump_moe_stage_probe_summary
 * (include/qx_format.h:160-161), same prototypes: the single-token attention stage
 * (src/qx_format.c:5478-5586) and the MoE stage (src/qx_format.c:5588-5725) of one layer
 * on a sidecar input, writing the reference's sidecars (<dir>/<name>-<layer>.f32) and JSON;
 * the stage arithmetic runs on the GPU (qxg_attention_stage, qxg_moe_stage). */
int qx_dump_attention_stage_probe_summary(const char *path, uint32_t layer, const char *layer_input_path,
        const char *output_dir, const char *activation_mode, const char *kv_format, FILE *out, char *err,
        uint64_t err_len);
int qx_dump_moe_stage_probe_summary(const char *path, uint32_t layer, const char *ffn_input_path,
        const char *output_dir, const char *activation_mode, FILE *out, char *err, uint64_t err_len);

#ifdef __cplusplus
}
#endif
#endif
