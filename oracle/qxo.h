/* ORACLE — test infrastructure only.  A scalar CPU restatement of the reference's
 * f32 decode path (reference src/qx_format.c), used by tests/, smoke() and the
 * cpu_baseline leg of bench.py as the checker.  The product path never links it.
 *
 * Every function cites the reference lines it restates.  Numeric contract
 * ("f32" activation mode): weights decode to f32 with the reference's op order,
 * products widen to double and accumulate in double in index order, results
 * narrow to float.  "q8_k_compat" mode: integer dots against Q8_K activations with
 * the reference's float scaling order. */
#ifndef QXO_H
#define QXO_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qxo_model qxo_model;

float qxo_fp16_to_f32(uint16_t h);
/* 256 values of one block of ggml type 12/14/17/18/23; returns 0 on unknown type */
int qxo_decode_block(uint32_t ggml_type, const uint8_t *raw, float out[256]);
uint64_t qxo_fnv1a64(const void *p, uint64_t n);

qxo_model *qxo_open(const char *path);            /* NULL on failure */
void qxo_close(qxo_model *m);
const uint8_t *qxo_tensor(const qxo_model *m, const char *name, uint32_t *type, uint64_t dims[4], uint64_t *bytes);

/* primitives */
void qxo_rmsnorm(const float *x, const float *w, float *y, uint32_t n, double *rms_out);
void qxo_head_rmsnorm(float *v, const float *w, uint32_t heads, uint32_t head_dim);
void qxo_rope(float *v, uint32_t heads, uint32_t head_dim, uint32_t pos, double theta);
float qxo_quantize_int8(const float *src, int8_t *dst, uint32_t n);
/* y[r] = (float) sum double(w) * double(x); non-finite -> 0 */
void qxo_matvec(uint32_t ggml_type, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y);

/* q8_k_compat activation mode (reference src/qx_format.c:3869-4205): activations
 * quantized to Q8_K blocks and integer dots per weight type.  The layout is ggml's
 * block_q8_K (292 bytes). */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } qxo_q8k;
/* 0 when n is not a multiple of 256 or a value is not finite */
int qxo_quantize_q8k(const float *x, uint32_t n, qxo_q8k *out);
/* rows of type t against x quantized to Q8_K (in_dims <= 4096); expert != 0: a
 * non-finite row fails (returns 0), else it is stored as 0 */
int qxo_matvec_q8k(uint32_t ggml_type, const uint8_t *w, uint32_t rows, uint32_t in_dims, const float *x, float *y,
                   int expert);
/* 0: f32 (default), 1: q8_k_compat for the attention projections, experts and head */
void qxo_set_activation(qxo_model *m, int q8_k_compat);

/* Q6_K head on a residual: output_norm then 151936 (vocab) rows; top_n <= 32 ids
 * ordered by (double logit desc, index asc).  Returns 0 on a non-finite logit. */
int qxo_final_head(qxo_model *m, const float *residual, float *norm_out, float *logits,
                   uint32_t top_n, uint32_t *top_ids, double *top_logits);

/* MoE block on ffn_inp: writes layer_out = ffn_inp + moe (and moe_out if non-NULL). */
int qxo_moe_layer(qxo_model *m, uint32_t layer, const float *ffn_inp, float *layer_out, float *moe_out,
                  uint32_t ids[8], double weights[8]);

/* Attention block for one token at `pos`: attn RMSNorm, K/V projection, k norm +
 * RoPE, INT8 quantize + store at [layer][pos], then Q projection/norm/RoPE, GQA
 * softmax over positions 0..pos and the O projection.  attn_out = O·ctx (no
 * residual).  kcache/vcache are [layers][ctx][512] int8, scales [layers*ctx]. */
int qxo_attention_layer(qxo_model *m, uint32_t layer, uint32_t pos, uint32_t ctx,
                        const float *x_in, int8_t *kcache, int8_t *vcache, float *kscales, float *vscales,
                        float *attn_out, float *kqv_out, float *vcur_out);

/* qxo_attention_layer plus the position's computed INT8 K/V row (row_k, row_v: 512
 * codes each; row_scales: k and v scale; each may be NULL); keep_row != 0 leaves the
 * cache's row at [layer][pos] unchanged and attends to it (same-input replay of a
 * device's attention on the device's own cache rows). */
int qxo_attention_layer_ex(qxo_model *m, uint32_t layer, uint32_t pos, uint32_t ctx,
                           const float *x_in, int8_t *kcache, int8_t *vcache, float *kscales, float *vscales,
                           float *attn_out, float *kqv_out, float *vcur_out,
                           int keep_row, int8_t *row_k, int8_t *row_v, float *row_scales);

/* One full token: embedding (Q4_K row), layers [0, layers), optional head.
 * layer_out (may be NULL) receives layers x 2048 floats of per-layer outputs. */
int qxo_decode_token(qxo_model *m, uint32_t token, uint32_t pos, uint32_t ctx, uint32_t layers,
                     int8_t *kcache, int8_t *vcache, float *kscales, float *vscales,
                     float *residual_out, float *layer_out, int run_head, float *logits,
                     uint32_t top_n, uint32_t *top_ids, double *top_logits);

/* Decodes the Q4_K embedding row of `token` (reference src/qx_format.c:3759-3793). */
int qxo_embed(qxo_model *m, uint32_t token, float *x);

/* f32 -> binary16 bits, round to nearest even (reference src/qx_format.c:1878-1902) */
uint16_t qxo_f32_to_fp16(float f);

/* attention stage probe (reference src/qx_format.c:5478-5586) of one layer input x:
 * norm[2048], vcur[512], kqv[4096], attn_out[2048], ffn_inp[2048]; probes: the V and O
 * row-dot sums.  f16_kv: the context takes an fp16 round trip. */
int qxo_attention_stage(qxo_model *m, uint32_t layer, const float *x, int f16_kv, float *norm, float *vcur,
                        float *kqv, float *attn_out, float *ffn_inp, double probes[2]);

/* MoE stage probe (reference src/qx_format.c:5588-5725) of one ffn input x.  out holds,
 * in order (E = experts, intermediate 768): ffn_norm[2048], logits[E], probs[E],
 * topk[8] (ids as floats), weights[8], weights_sum[1], weights_norm[8], gate[8*768],
 * up[8*768], swiglu[8*768], down[8*2048], weighted[8*2048]. */
#define QXO_MOE_STAGE_FLOATS(E) (2048u + 2u * (E) + 25u + 3u * 8u * 768u + 2u * 8u * 2048u)
int qxo_moe_stage(qxo_model *m, uint32_t layer, const float *x, float *out, uint32_t ids[8]);

#ifdef __cplusplus
}
#endif
#endif
