/* qxg — C ABI to the MI355X (gfx950) decode path.
 *
 * The reference has no process or device boundary: its state loop calls static
 * C functions over mmap'd weight spans (reference src/qx_format.c:5970-6733).  This
 * ABI is the seam that replaces those calls.  Each entry point below names the
 * reference function(s) it stands in for.  Conventions follow the reference C API
 * (reference include/qx_format.h:104-172): return 1 on success and 0 on failure,
 * with a message written into (err, err_len).  Pointers are host pointers, sizes
 * are plain integers, and calls are synchronous unless stated otherwise.  Each
 * context owns one HIP stream and its device buffers.  A context is not
 * thread-safe (the reference is single-threaded, src/qx_format.c:5984-5995).
 *
 * Fixed model geometry (reference --final-head manifest check,
 * src/qx_format.c:6120-6124): hidden 2048, 32 q heads / 4 kv heads of 128,
 * moe_intermediate 768, top-8 experts; vocab, experts (8..128) and layer count
 * come from the uploaded tensors.
 */
#ifndef QXG_H
#define QXG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qxg_ctx qxg_ctx;

/* Creates a context on HIP device `device`: stream, codebooks, RoPE table.
 * Stands in for the per-call setup of the reference state loop
 * (src/qx_format.c:6044-6160). */
int qxg_open(int device, qxg_ctx **out, char *err, uint64_t err_len);
void qxg_close(qxg_ctx *ctx);

/* Uploads one tensor of the QXF1 file (bytes = the tensor's mmap span) and repacks
 * quantized blocks on the device.  Replaces the per-call weight reads
 * qx_read_raw_span / qx_acquire_span (src/qx_format.c:1757-1773, 858-893).
 * ggml_type: 0 F32, 12 Q4_K, 13 Q5_K, 14 Q6_K, 17 IQ2_XS, 18 IQ3_XXS, 21 IQ3_S,
 * 22 IQ2_S, 23 IQ4_XS. */
int qxg_upload_tensor(qxg_ctx *ctx, const char *name, uint32_t ggml_type, const uint64_t dims[4],
                      const void *host_bytes, uint64_t nbytes, char *err, uint64_t err_len);

/* Resolves the uploaded tensors into layers [0, layers), checks every shape and
 * type (the checks of src/qx_format.c:5216-5235, 3610-3629), and sizes work
 * buffers.  need_head / need_embedding select whether output.* / token_embd.* must
 * be present.  Per layer: attn_q/k/v/output IQ4_XS or Q5_K; gate/up experts IQ2_XS
 * or IQ2_S (both the same); down experts IQ3_XXS, IQ4_XS or IQ3_S.  A model using any
 * format beyond IQ4_XS / IQ2_XS / IQ3_XXS decodes one kernel per phase; its prefill
 * (qxg_prefill / qxg_prefill_layer) stays batched on the matrix cores. */
int qxg_bind_model(qxg_ctx *ctx, uint32_t layers, int need_embedding, int need_head, char *err, uint64_t err_len);

/* Persistent INT8 KV cache [layers][ctx_tokens][512] for K and V plus one f32 scale
 * per (layer, position).  Same layout as the reference state loop
 * (src/qx_format.c:6138-6160, 6343-6400).  kv_format must be 1 (int8). */
int qxg_kv_create(qxg_ctx *ctx, uint32_t layers, uint32_t ctx_tokens, uint32_t kv_format, char *err, uint64_t err_len);
/* Copies rows [pos0, pos0+count) of one layer into / out of the device cache.
 * k, v: count*512 int8; kscale, vscale: count floats.  Used for QXKVSNP1
 * import/export (src/qx_format.c:5860-5968) and for seeded long-context tests. */
int qxg_kv_write(qxg_ctx *ctx, uint32_t layer, uint32_t pos0, uint32_t count, const int8_t *k, const int8_t *v,
                 const float *kscale, const float *vscale, char *err, uint64_t err_len);
int qxg_kv_read(qxg_ctx *ctx, uint32_t layer, uint32_t pos0, uint32_t count, int8_t *k, int8_t *v,
                float *kscale, float *vscale, char *err, uint64_t err_len);

/* QXKVSNP1 snapshots of the INT8 KV cache (the reference's accumulated-KV files,
 * qx_write_accumulated_kv_snapshot / qx_read_accumulated_kv_snapshot,
 * src/qx_format.c:5860-5968, used by --kv-snapshot-out / --kv-snapshot-in,
 * src/qx_format.c:6165-6177, 6629-6633).  File: 48-byte header ("QXKVSNP1", version 2,
 * layers, positions, ctx_tokens, kv_heads 4, head_dim 128, format 1 = int8, row bytes
 * 512, next_token, seed), per layer and position the K row, V row, K scale and V scale,
 * then the SHA-256 of all preceding bytes.  ctx_tokens must equal the cache's context.
 * qxg_kv_export writes layers [0, layers) x positions [0, positions) of the device cache;
 * qxg_kv_import checks the header (layers, ctx_tokens, kv geometry, int8, seed) and the
 * digest before writing positions [0, *positions_out) of every layer to the device. */
int qxg_kv_export(qxg_ctx *ctx, const char *path, uint32_t layers, uint32_t positions, uint32_t ctx_tokens,
                  uint32_t next_token, uint32_t seed, char *err, uint64_t err_len);
int qxg_kv_import(qxg_ctx *ctx, const char *path, uint32_t layers, uint32_t ctx_tokens, uint32_t seed,
                  uint32_t *positions_out, uint32_t *next_token_out, char *err, uint64_t err_len);
/* The same file format over host caches laid out as the reference's
 * ([layers][ctx_tokens][512] int8 rows, [layers*ctx_tokens] f32 scales); no device use. */
int qxg_kvsnap_write(const char *path, uint32_t layers, uint32_t positions, uint32_t ctx_tokens, uint32_t next_token,
                     uint32_t seed, const int8_t *k, const int8_t *v, const float *kscale, const float *vscale,
                     char *err, uint64_t err_len);
int qxg_kvsnap_read(const char *path, uint32_t layers, uint32_t ctx_tokens, uint32_t seed, int8_t *k, int8_t *v,
                    float *kscale, float *vscale, uint32_t *positions_out, uint32_t *next_token_out, char *err,
                    uint64_t err_len);

/* One full token at `position`: Q4_K embedding, every bound layer (attention with
 * INT8 KV append, then MoE), and if run_head the output RMSNorm, Q6_K head and
 * top_n (<= 32) ids by (logit desc, index asc).  The loop body of
 * qx_dump_prompt_state_loop_probe_summary (src/qx_format.c:6250-6627).
 * Any output pointer may be NULL.  layer_out: layers*2048 floats (the per-layer
 * "output" residual dumps, src/qx_format.c:6439).  Returns 0 on a non-finite
 * logit (src/qx_format.c:3715). */
int qxg_decode_token(qxg_ctx *ctx, uint32_t token, uint32_t position, int run_head,
                     float *residual_out, float *layer_out, float *logits, uint32_t top_n,
                     uint32_t *top_ids, double *top_logits, char *err, uint64_t err_len);

/* Greedy loop on the device: feeds prompt[0..n_prompt) at positions pos0.., then
 * generates n_gen tokens by argmax with the next token fed back on the device
 * (no host round trip per step).  tokens_out receives the n_gen generated ids.
 * Matches the step/phase sequence of src/qx_format.c:6250-6627 with temperature 0
 * (qx_sample_from_top, src/qx_format.c:3045-3057).  If elapsed_ms is non-NULL it
 * receives the device time of the whole loop (HIP events on the context stream). */
int qxg_generate(qxg_ctx *ctx, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_gen, uint32_t pos0,
                 uint32_t *tokens_out, float *elapsed_ms, char *err, uint64_t err_len);

/* 1 when qxg_generate / qxg_decode_token run the persistent decode on this context (the
 * layer path set to 1, the f32 activation mode, every bound format one it decodes), else 0.
 * No reference counterpart. */
int qxg_persistent_path(const qxg_ctx *ctx);

/* qxg_generate with every step's records, for the reference's prompt state loop
 * (qx_dump_prompt_state_loop_probe_summary, src/qx_format.c:6250-6627, which prints them per
 * step and layer): one persistent launch over the S = n_prompt + n_gen - 1 steps, then the
 * top_n (<= 32) tokens of each head step ranked on the device and everything copied back in
 * bulk.  Persistent path only (qxg_persistent_path); the records live in device buffers
 * allocated for the call.  Outputs, any of which may be NULL, with L = the bound layers:
 *   tokens_out[S + 1]      the prompt, then each generated id at [step + 1];
 *   layer_out[S][L][2048]  each layer's output residual;
 *   attn_out, moe_out      [S][L][2048] each layer's attention output and MoE sum (before
 *                          their residual adds, as qxg_decode_halves);
 *   ids_out, weights_out   [S][L][8] the routing (as qxg_decode_routing);
 *   head_sums_out[S][L][32] each q head's sum of normalised attention weights;
 *   norm_out[S][2048], logits_out[S][vocab]   each head step's output-RMSNorm vector and
 *                          logits (steps before the last prompt token run no head: zeros);
 *   top_ids, top_logits    [S][top_n] each head step's best tokens, highest first (zeros
 *                          before the last prompt token);
 *   step_ms[S + 1]         the device clock at each step's start and at the end, in ms from
 *                          the first step's start;
 *   elapsed_ms             the device time of the launch (HIP events).
 * Returns 0 on a non-finite final logit (src/qx_format.c:3715) or a bad argument. */
int qxg_generate_recorded(qxg_ctx *ctx, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_gen, uint32_t pos0,
                          uint32_t top_n, uint32_t *tokens_out, float *layer_out, float *attn_out, float *moe_out,
                          uint32_t *ids_out, double *weights_out, double *head_sums_out, float *norm_out, float *logits_out,
                          uint32_t *top_ids, double *top_logits, double *step_ms, float *elapsed_ms, char *err,
                          uint64_t err_len);

/* ---- same-input replay seams (host pointers in and out, synchronous) ---- */

/* Q4_K embedding row of `token` as 2048 floats, no norm on the full-MoE path:
 * replaces qx_fill_residual_vector_from_embedding (src/qx_format.c:3759-3793). */
int qxg_embed_token(qxg_ctx *ctx, uint32_t token, float *x_out, char *err, uint64_t err_len);

/* Decodes `nblocks` consecutive 256-value blocks of one type to f32, on the
 * device, from the repacked layout, with the reference's op order (bit-exact with
 * qx_decode_supported_block, src/qx_format.c:2206-2217). */
int qxg_dequant_blocks(qxg_ctx *ctx, uint32_t ggml_type, const void *raw, uint64_t nblocks, float *out,
                       char *err, uint64_t err_len);

/* INT8 KV quantization of one row of n <= 4096 f32 values on the device, with the same
 * device functions every kernel that appends a KV row uses: scale = max|x| / 127 over the
 * finite values (1 if zero), codes = lrintf(x / scale) clamped to +-127, non-finite -> 0.
 * Replaces qx_quantize_int8_vector (src/qx_format.c:4449-4463) as a same-input seam. */
int qxg_int8_quantize(qxg_ctx *ctx, const float *x, uint32_t n, int8_t *codes, float *scale, char *err, uint64_t err_len);

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * qxg_dequant_blocks with the raw blocks and the f32 output in device memory the caller
 * owns (raw_dev: nblocks blocks of the type's size; out_dev: nblocks * 256 floats) and
 * the repacked block planes in a static device workspace (one per GPU, held until the
 * process ends) instead of per-call allocations.  At most QXG_STATIC_MAX_BLOCKS blocks
 * per call; more fail with an error.  Allocates nothing; returns when the output is
 * written.  Every call on one GPU shares its workspace: calls that overlap on one GPU
 * (from several threads or contexts) are serialised by a per-GPU lock held from the
 * repack until the call has finished. */
#define QXG_STATIC_MAX_BLOCKS 4096u
int qxg_dequant_blocks_static(qxg_ctx *ctx, uint32_t ggml_type, const void *raw_dev, uint64_t nblocks, float *out_dev,
                              char *err, uint64_t err_len);

/* Attention block of `layer` for one token at `position` on residual x_in:
 * attn RMSNorm, K/V projections, k norm + RoPE, INT8 append at [layer][position],
 * Q projection/norm/RoPE, GQA softmax over 0..position, O projection.
 * attn_out = O*ctx (without the residual).  Replaces the attention half of the
 * layer loop (src/qx_format.c:6282-6423 and qx_rope_gqa_attention_partial,
 * 5051-5196).  kqv_out: 4096 floats, vcur_out: 512 floats (dump phases
 * "kqv-out" and "v-cur"). */
int qxg_attention_layer(qxg_ctx *ctx, uint32_t layer, uint32_t position, const float *x_in, float *attn_out,
                        float *kqv_out, float *vcur_out, char *err, uint64_t err_len);
/* qxg_attention_layer plus, when head_weight_sums is non-NULL, each q head's sum of its
 * normalised softmax weights (32 doubles): the reference reports their mean, minimum and
 * maximum as softmax_sum, softmax_sum_min, softmax_sum_max (src/qx_format.c:5154-5189,
 * printed at 6516-6523). */
int qxg_attention_layer_ex(qxg_ctx *ctx, uint32_t layer, uint32_t position, const float *x_in, float *attn_out,
                           float *kqv_out, float *vcur_out, double *head_weight_sums, char *err, uint64_t err_len);

/* The attention stage probe's computation (qx_dump_attention_stage_probe_summary,
 * src/qx_format.c:5478-5586): a single token attending to itself.  attn RMSNorm (norm_out,
 * 2048), V projection (vcur_out, 512), each q head's context = its kv head's V row, after
 * an fp16 round trip if f16_kv (kqv_out, 4096), O projection (attn_out, 2048), ffn_inp_out =
 * x_in + attn_out.  Fails with the reference's message on a non-finite output.  Output
 * pointers may be NULL. */
int qxg_attention_stage(qxg_ctx *ctx, uint32_t layer, int f16_kv, const float *x_in, float *norm_out,
                        float *vcur_out, float *kqv_out, float *attn_out, float *ffn_inp_out, char *err,
                        uint64_t err_len);

/* The MoE stage probe's computation (qx_dump_moe_stage_probe_summary, src/qx_format.c:
 * 5588-5725) on ffn input x_in: f32 router logits, f32 softmax probabilities, 8 picks by
 * probability, f32 renormalised weights, then per pick the gate, up, SwiGLU, down and
 * weighted down rows.  out receives QXG_MOE_STAGE_FLOATS(experts) floats, in order:
 * ffn_norm[2048], logits[E], probs[E], topk[8] (ids as floats), weights[8],
 * weights_sum[1], weights_norm[8], gate[8][768], up[8][768], swiglu[8][768],
 * down[8][2048], weighted[8][2048]; ids (may be NULL) the picks. */
#define QXG_MOE_STAGE_FLOATS(E) (2048u + 2u * (E) + 25u + 3u * 8u * 768u + 2u * 8u * 2048u)
int qxg_moe_stage(qxg_ctx *ctx, uint32_t layer, const float *x_in, float *out, uint32_t ids[8], char *err,
                  uint64_t err_len);

/* MoE block of `layer` on ffn_inp: replaces qx_apply_real_moe_layer
 * (src/qx_format.c:5198-5317).  layer_out = ffn_inp + moe; moe_out (may be NULL)
 * = the "ffn-moe-out" dump; ids/weights = selected experts in rank order. */
int qxg_moe_layer(qxg_ctx *ctx, uint32_t layer, const float *ffn_inp, float *layer_out, float *moe_out,
                  uint32_t ids[8], double weights[8], char *err, uint64_t err_len);

/* Output head on a residual: replaces qx_compute_real_final_head
 * (src/qx_format.c:3554-3738) as used by qx_dump_final_head_probe_summary
 * (src/qx_format.c:5369-5411).  norm_out: 2048 floats, logits: vocab floats. */
int qxg_final_head(qxg_ctx *ctx, const float *residual, float *norm_out, float *logits, uint32_t top_n,
                   uint32_t *top_ids, double *top_logits, char *err, uint64_t err_len);

/* Batched prefill: tokens[0..n) at positions position0.. through every bound layer
 * together (projection and expert GEMMs on the matrix cores), INT8 KV appended at
 * [layer][position0+i]; then, if run_head, the output RMSNorm, Q6_K head and top_n on
 * the last token.  Stands in for the reference's prompt steps, which run one token at a
 * time through the decode step with the head only on the last prompt token
 * (src/qx_format.c:6250-6547, sampling_step at 6253).  Chunks of 512 tokens run in
 * order; every per-layer format of the real checkpoint (IQ4_XS / Q5_K attention,
 * IQ2_XS / IQ2_S gate/up, IQ3_XXS / IQ3_S / IQ4_XS down) runs batched.  The q8_k_compat
 * mode takes those token steps on the device instead: one persistent launch over the
 * prompt where the persistent path serves the model and residual_out is NULL, else the
 * one-kernel-per-phase decode kernels one token at a time; either way the result equals
 * qxg_decode_token over the prompt on the same layer path.
 * residual_out (may be NULL): n*2048 floats, each token's residual after the
 * last layer.  logits / top_* as in qxg_decode_token.  elapsed_ms: device time of the
 * whole call (HIP events on the context stream). */
int qxg_prefill(qxg_ctx *ctx, const uint32_t *tokens, uint32_t n, uint32_t position0, int run_head,
                float *residual_out, float *logits, uint32_t top_n, uint32_t *top_ids, double *top_logits,
                float *elapsed_ms, char *err, uint64_t err_len);

/* Same-input replay of one prefill layer: n <= 512 residual rows x_in (n*2048) at
 * positions position0.. (KV rows appended as in qxg_prefill).  ffn_inp_out = x_in +
 * attention (the MoE input, dump phase "ffn-inp"), moe_out = the weighted expert sum
 * ("ffn-moe-out"), x_out = ffn_inp + moe; any output may be NULL.  The reference's
 * counterpart is n successive layer steps (src/qx_format.c:6282-6423, 5198-5317). */
int qxg_prefill_layer(qxg_ctx *ctx, uint32_t layer, uint32_t n, uint32_t position0, const float *x_in,
                      float *ffn_inp_out, float *moe_out, float *x_out, char *err, uint64_t err_len);

/* How the layers of a token are launched (no reference counterpart: the reference
 * runs one thread on the CPU).  1 (the default): one cooperative persistent kernel per
 * qxg_generate / qxg_decode_token call runs every step (embedding, all layers, head,
 * argmax), one workgroup per CU, its phases handed over through epoch-tagged device
 * words; 0: one kernel per phase, six per layer, each step replayed from a recorded
 * graph.  Both give the same results to the stated tolerance.  Drops the recorded decode
 * graph.  A model bound with formats beyond IQ4_XS / IQ2_XS / IQ3_XXS runs path 0
 * whatever is set here; the q8_k_compat mode runs either path (the persistent kernel has
 * a Q8_K instantiation). */
int qxg_set_layer_path(qxg_ctx *ctx, int persistent);

/* Activation format of the projections, experts and head: 0 "f32" (default), 1
 * "q8_k_compat" -- the reference's activation_format argument of the state loop and
 * stage probes (src/qx_format.c:5970-5972, 4217-4218, 5286-5288, 3565).  In
 * q8_k_compat the matvec inputs are quantized to Q8_K blocks (256 values, one f32
 * scale) and each weight type is dotted in integers; a non-finite activation or
 * expert row makes the call fail with the reference's message.  Decode follows
 * qxg_set_layer_path (the persistent kernel's Q8_K instantiation by default);
 * qxg_prefill runs token by token through the one-kernel-per-phase decode kernels in
 * this mode.  Drops the recorded decode graph. */
int qxg_set_activation(qxg_ctx *ctx, uint32_t activation_format, char *err, uint64_t err_len);

/* Routing of every layer in the last step run by qxg_decode_token (or the last step of
 * qxg_generate): ids[l*8 + r] the expert of rank r in layer l, weights[l*8 + r] its
 * renormalised weight, as qx_apply_real_moe_layer selects them (src/qx_format.c:5265-5290).
 * The reference keeps no such record; this is the readback the router parity tests use. */
int qxg_decode_routing(qxg_ctx *ctx, uint32_t layers, uint32_t *ids, double *weights, char *err, uint64_t err_len);

/* The two halves of every layer in the last step run by qxg_decode_token, before their
 * residual adds: attn_out[l*2048 ..] the attention output (the O projection of the
 * context; the reference's "attn-out" dump phase, src/qx_format.c:6420-6423) and
 * moe_out[l*2048 ..] the weighted expert sum ("ffn-moe-out", :5296-5309).  Either may be
 * NULL.  Same-input replay of each half on its own: the residual stream can be many orders
 * of magnitude larger than a half, so a layer output alone would hide an error in it. */
int qxg_decode_halves(qxg_ctx *ctx, uint32_t layers, float *attn_out, float *moe_out, char *err, uint64_t err_len);

/* Persistent decode only (no reference counterpart): from n = position + 1 >=
 * min_positions on, stage A attends by (kv head, 64-position chunk) over every workgroup
 * and merges the chunks' partial softmax results; below it the 32 q-head workgroups walk
 * the cache themselves.  Default 577 (measured crossover of the two); 1 chunks every position,
 * 4097 never. */
int qxg_set_attention_chunks(qxg_ctx *ctx, uint32_t min_positions);

/* The output-RMSNorm vector (2048 floats) of the last head step run by qxg_decode_token:
 * the normalised final residual the head consumed (src/qx_format.c:3655, the state loop's
 * final_norm_raw). */
int qxg_decode_final_norm(qxg_ctx *ctx, float *norm_out, char *err, uint64_t err_len);

/* Each q head's sum of its normalised attention weights in every layer of the last step run
 * by qxg_decode_token: sums[l*32 + h].  The state loop's per-layer softmax_sum fields
 * (src/qx_format.c:5183-5190, printed at :6494-6529); the reference keeps no other record. */
int qxg_decode_head_sums(qxg_ctx *ctx, uint32_t layers, double *sums, char *err, uint64_t err_len);

/* The cache rows of one position in layers [0, layers): k, v layers*512 int8 and the
 * scales, one strided copy each (qxg_kv_read per layer, batched for the state loop's
 * per-step K/V checksums, src/qx_format.c:6494-6529). */
int qxg_kv_read_position(qxg_ctx *ctx, uint32_t position, uint32_t layers, int8_t *k, int8_t *v, float *ks, float *vs,
                         char *err, uint64_t err_len);

/* Same-input seam of the Q8_K quantizer the q8_k_compat kernels use: n values (a
 * multiple of 256, at most 4096) -> n/256 blocks of 292 bytes in ggml's block_q8_K
 * layout {f32 d, int8 qs[256], int16 bsums[16]}.  Replaces qx_quantize_q8_k as exposed
 * by the reference's q8-k-activation-probe (src/qx_format.c:3891-3927, 4304-4345);
 * fails, like it, on a non-finite value or a bad length. */
int qxg_q8k_quantize(qxg_ctx *ctx, const float *x, uint32_t n, void *blocks_out, char *err, uint64_t err_len);

/* ---- measurement (no reference counterpart: the reference times with clock(),
 *      src/qx_format.c:6245, 6642-6653) ---- */

/* Average device time (ms) of one launch of kernel `which` over `iters` launches,
 * bracketed by HIP events on the context stream.  which: 0 gate/up experts,
 * 1 down experts, 2 Q/K/V projection, 3 O projection, 4 Q6_K head, 5 attention,
 * 6 router.  Uses layer `layer`'s weights and the current routing/KV state. */
int qxg_time_kernel(qxg_ctx *ctx, int which, uint32_t layer, uint32_t iters, float *avg_ms, char *err, uint64_t err_len);
/* Device bytes held by uploaded tensors (repacked; equal to the QXF1 tensor bytes). */
uint64_t qxg_device_bytes(const qxg_ctx *ctx);
/* In-situ timing: while enabled, qxg_generate / qxg_decode_token record a HIP
 * event pair around every launch of kernel `which` (numbering of
 * qxg_time_kernel, plus 7 the persistent layer kernel and, for qxg_prefill, 8 Q/K/V,
 * 9 O, 10 gate/up and 11 down GEMMs, 12 router logits, 13 attention; -1 disables).
 * qxg_profile_result sums the pairs. */
int qxg_profile_kernel(qxg_ctx *ctx, int which);
int qxg_profile_result(qxg_ctx *ctx, uint32_t *launches, double *total_ms);

#ifdef __cplusplus
}
#endif
#endif
