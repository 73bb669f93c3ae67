// Internal declarations shared by the device kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QXG_HIDDEN 2048
#define QXG_QDIM 4096
#define QXG_KVDIM 512
#define QXG_HEADS 32
#define QXG_KVHEADS 4
#define QXG_HEAD_DIM 128
#define QXG_FFN 768
#define QXG_TOPK 8
#define QXG_MAX_CTX 4096
#define QXG_MAX_TOPN 32

// Repacked quantized tensor: every field of the original block in its own array,
// so each lane's load is aligned.  Bytes per block are unchanged.
//   IQ4_XS : qs[nb][128], meta[nb][8] = {d, scales_h, scales_l[4]}
//   IQ2_XS : qs[nb][64] (32 x u16), sc[nb][8], d[nb]
//   IQ3_XXS: qs[nb][64], aux[nb][32] (8 x u32), d[nb]
//   Q6_K   : ql[nb][128], qh[nb][64], sc[nb][16] (int8), d[nb]
//   Q5_K   : qs[nb][128], meta[nb][16] = {d, dmin, scales[12]}, qh[nb][32]
//   IQ2_S  : qs[nb][64] (32 grid bytes, 32 sign bytes), sc[nb][8], qh[nb][8], d[nb]
//   IQ3_S  : qs[nb][64], signs[nb][32], {qh[8], scales[4], 0[4]}[nb], d[nb]
//   Q4_K, F32: the original bytes
struct QTensor {
    uint32_t type = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t nblocks = 0, bytes = 0;
    uint8_t *base = nullptr;      // device allocation
    const uint8_t *p0 = nullptr;  // qs / ql / raw
    const uint8_t *p1 = nullptr;  // meta / sc / aux / qh / signs
    const uint8_t *p2 = nullptr;  // Q6_K sc, Q5_K qh, IQ2_S qh, IQ3_S qh+scales
    const uint16_t *d = nullptr;  // fp16 d per block
};

struct LayerW {
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm, *router;
    const QTensor *wq, *wk, *wv, *wo, *gate, *up, *down;
};

// Device-resident step state: kernels read the position from here so one
// recorded step can be replayed for every token.
struct DevState {
    uint32_t pos0;          // position of local step 0
    uint32_t step;          // local step
    uint32_t n_prompt;      // steps < n_prompt-1 are prompt steps (no head)
    uint32_t nonfinite;     // set by the head on a non-finite logit
    uint32_t spare;         // unused (keeps the layout of the host-written prefix)
    uint32_t spare2;        // unused (keeps the layout of the host-written prefix)
    uint32_t force_head;    // run the head on every step
    uint32_t pad;
    uint32_t moe_ids[QXG_TOPK];
    double moe_w[QXG_TOPK];
    uint32_t epoch;         // unused (keeps the layout)
    uint32_t q8_fault;      // q8_k_compat failure of the step (QXG_Q8_*), cleared by the host
    double rope_c[64];      // RoPE cos/sin row of the current position (pos0 + step), written
    double rope_s[64];      // with the position by the host and by qxk_advance
};

// q8_k_compat failures, reported as the reference reports them (src/qx_format.c:3906, 4771)
#define QXG_Q8_NONFINITE_INPUT 1u    // "Q8_K activation contains NaN or Inf"
#define QXG_Q8_NONFINITE_EXPERT 2u   // "non-finite packed expert Q8_K output"

struct Tables {
    uint4 *g2;     // IQ2_XS grid: 512 x {pos lo, pos hi, neg lo, neg hi}
    uint2 *g3;     // IQ3_XXS grid: 256 x {pos, neg}
    uint2 *sel;    // sign index (7 bits) -> v_perm selectors for 8 values
    double *rope_cos, *rope_sin;  // [QXG_MAX_CTX][64]
    double *rope_cs;              // [QXG_MAX_CTX][128]: the position's 64 cos, then its 64 sin
    uint4 *g2s;    // IQ2_S grid: 1024 x {pos lo, pos hi, neg lo, neg hi}
    uint2 *g3s;    // IQ3_S grid: 512 x {pos, neg}
    uint2 *sel8;   // sign byte (8 bits) -> v_perm selectors for 8 values
};

// Decode attention splits: a block takes QXG_ATT_SPLIT positions of one q head; the
// per-split results (128 context sums, then the maximum score and the exp-sum as
// doubles) are QXG_ATT_PART floats, at [head][split].
#define QXG_ATT_SPLIT 128
#define QXG_MAX_SPLITS (QXG_MAX_CTX / QXG_ATT_SPLIT)
#define QXG_ATT_PART 132
#define QXG_ATT_PART_BYTES (32 * QXG_MAX_SPLITS * QXG_ATT_PART * 4)

// Rows (units) per wave of the decode matvec kernels.  A wave's gate/up units must lie
// in one expert (UPW | 768).
#ifndef QXG_GU_UPW
#define QXG_GU_UPW 3
#endif
#ifndef QXG_OPROJ_RPW
#define QXG_OPROJ_RPW 2
#endif
#ifndef QXG_DOWN_RPW
#define QXG_DOWN_RPW 2
#endif
static_assert(768 % QXG_GU_UPW == 0, "a wave's units must not straddle an expert");

// Persistent decode kernel (qxk_decode): per-layer weight pointers and launch arguments.
#define QXG_PBLOCKS 256   // workgroups of the persistent decode kernel: one per CU of an MI355X

// One plane of a per-layer tensor kind: the planes of all layers lie back to back in
// one device arena, layer l's at base + l * stride, so a kernel forms every layer's
// pointers with scalar arithmetic on its arguments (no pointer-table loads).
struct QxPlane {
    const uint8_t *base;
    uint64_t stride;
};
enum QxPlaneId : int {
    PL_ATTN_NORM, PL_Q_NORM, PL_K_NORM, PL_FFN_NORM, PL_ROUTER,   // F32
    PL_Q_QS, PL_Q_META, PL_K_QS, PL_K_META, PL_V_QS, PL_V_META,    // IQ4_XS
    PL_O_QS, PL_O_META,
    PL_G_QS, PL_G_SC, PL_G_D, PL_U_QS, PL_U_SC, PL_U_D,            // IQ2_XS
    PL_D_QS, PL_D_AUX, PL_D_D,                                     // IQ3_XXS
    PL_COUNT
};

// Arguments of the persistent decode kernel qxk_decode (qxg_decode.hip), built by the host
// for the benchmark quant mix.
struct QxDArgs {
    QxPlane P[PL_COUNT];         // per-layer weight planes (layer l at base + l * stride)
    QxPlane GU;                  // routed experts' gate/up rows, unit-interleaved (QXD_GU_UNIT bytes per unit)
    QxPlane DN;                  // routed experts' down rows (QXD_DN_ROW bytes per row), 8-row blocks of all experts together
    QxPlane PK;                  // each workgroup's dense rows of the layer (QXD_PK_*), 256 packs of QXD_PK_BYTES
    const uint8_t *emb;          // Q4_K token embedding
    uint64_t emb_row;
    const float *out_norm;
    const uint8_t *h_ql, *h_qh;  // Q6_K head planes
    const uint8_t *h_il;         // the head rows interleaved, QXD_HEAD_ROW bytes per row
    const int8_t *h_sc;
    const uint16_t *h_d;
    uint32_t vocab, layers, experts, ctx;
    uint32_t steps, n_prompt, pos0, force_head;
    uint32_t ep0;                // epoch base of the launch (its phases are ep0 + 1 ...)
    Tables T;
    int8_t *kc, *vc;
    float *ks, *vs;
    uint32_t *tokens;            // tokens[0 .. n_prompt) in; generated ids stored at [step + 1]
    DevState *st;                // nonfinite flag
    uint64_t *xch;               // tagged exchange buffers (QXD_XCH_WORDS words, zeroed once)
    uint64_t *xpart;             // tagged partial results of the chunked attention (2 QXD_PART_WORDS)
    float *logits;               // optional: the last head step's logits
    float *d_layer;              // optional dumps of the last step: per-layer output residuals,
    uint32_t *d_rids;            // routed experts and renormalised weights per layer, the
    double *d_rw;                // final residual, and each layer's two halves before their
    float *d_res;                // residual adds ([layer][attention 2048 | MoE 2048])
    float *d_half;
    double *d_wsum;              // [layer][32] each q head's sum of normalised attention weights
    float *d_norm;               // the last head step's output-RMSNorm vector (2048)
    uint32_t rec_all;            // 1: the dumps (and logits) of every step, at record slot rec_base + step
    uint32_t rec_base;           //    (dump arrays then hold one slot per step); 0: the last step's only
    uint64_t *d_time;            // optional with rec_all: 100 MHz clock at each step's start on workgroup 0
                                 //    ([rec_base + step]) and at the launch's end ([rec_base + steps])
    uint32_t *abort;             // set on a timed-out wait; the host reports it
    uint64_t timeout;            // per wait, in 100 MHz ticks
    double sqrt_hd;
};
#define QXD_THREADS 512
// Interleaved expert rows of the persistent decode: unit (expert e, row r) of gate/up is
// [gate qs 512 | sc 64 | d 16 | up qs 512 | sc 64 | d 16] at (e * 768 + r) * 1184; down row
// (e, r) is [qs 192 | aux 96 | d 6 | 0 x 10] at (((r / 8) * E + e) * 8 + r % 8) * 304 (the
// 8-row blocks of all E experts for one row range together).  A wave's rows then lie in one
// contiguous range, so each of its 16-byte load instructions touches one or two pages (the
// cost of a scattered load instruction grows with the pages it touches).
#define QXD_GU_UNIT 1184u
// Q6_K head row r of the persistent decode: [ql 1024 | qh 512 | sc 128 | d 16] at r * 1680
// (the 8 blocks' planes of the row back to back; 105 16-byte chunks).
#define QXD_HEAD_ROW 1680u
#define QXD_DN_ROW 304u
// Decode pack of workgroup w (0..255) for one layer: the dense rows it reads, copied
// contiguously so that its loads of a layer touch one or two translation pages instead of
// one per plane (Q/K/V, O, their metas, router, router fold).  Workgroups w >= 32 make the
// Q/K/V rows: 24 slots, slot 3 v + r = stacked row [Q 4096 | K 512 | V 512] 24 (w - 32) +
// 3 v + r (224 x 24 >= 5120; the slots past row 5119 are zero).  Byte offsets in the pack:
#define QXD_PK_QQ 0u        // the 24 Q/K/V slots' IQ4_XS qs (8 blocks x 128 B a row)
#define QXD_PK_OQ 24576u    // O rows 8 w .. 8 w + 7, qs (16 blocks x 128 B a row)
#define QXD_PK_QM 40960u    // the Q/K/V slots' 8-byte block metas
#define QXD_PK_OM 42496u    // the O rows' metas
#define QXD_PK_RT 43520u    // w < experts: router row W[w], 2048 f32
#define QXD_PK_MF 51712u    // w < experts: router fold row M[w], 4096 f32
#define QXD_PK_BYTES 68096u
// The four per-layer norm vectors share one arena: layer l's at l * QXD_NORM_STRIDE, attn
// norm (2048 f32) at 0, ffn norm at 8192, q norm (128 f32) at 16384, k norm at 16896.
#define QXD_NORM_STRIDE 17408u
// Long-context attention of the persistent decode: stage A by (kv head g, chunk c) of
// QXD_CHUNK positions, one workgroup each, then a merge by (q head, 16 dimensions).  A
// chunk's partial result for one q head and 16 dimensions is a record of QXD_PREC words
// {context sums 16, running maximum (hi, lo), denominator (hi, lo)} at
// [head][dimension group][chunk].
#define QXD_CHUNK 64u
#define QXD_CHUNK_S 32u          // ... of QXD_CHUNK_S positions while the cache has at most
#define QXD_CHUNK_S_MAXN 2048u   //     QXD_CHUNK_S_MAXN (more workgroups, each with less to do)
#define QXD_PREC 20u
#define QXD_PART_WORDS (32u * 8u * (QXG_MAX_CTX / QXD_CHUNK) * QXD_PREC)
// Default positions (n = pos + 1) from which the persistent decode attends by chunk: below
// it the 32 q-head workgroups walk the cache themselves (no merge exchange).
#define QXD_SPLIT_MIN_DEFAULT 577u
// exchange words per launch: x, qkv, ctx, x', router logits, h, expert weights (two slots
// each) and the per-workgroup argmax candidates; the chunked attention's partial results
// (two slots of QXD_PART_WORDS) have a buffer of their own
#define QXD_XCH_WORDS (2u * (2048u + 5120u + 4096u + 2048u + 256u + 6144u + 16u + 2u * QXG_PBLOCKS))
// phases per step (five exchanges per layer, the head input, the argmax)
#define QXD_PHASES(layers) (5u * (layers) + 2u)

// ---- batched prefill (qxg_prefill.hip)
#define QXP_MAX 512   // tokens per prefill chunk
// 32-row tiles per wave of the expert GEMMs.  One tile keeps a workgroup at 64 KiB of
// LDS and few enough registers for two workgroups per CU: gate/up 118 -> 102 us and
// down 87 -> 65 us per layer at T = 512 against two tiles (one workgroup per CU).
#define QXG_PF_EXPERT_MT 1

// fp16 codebooks of the prefill GEMMs (built on the host at first use)
struct PfTables {
    uint4 *g2h;      // IQ2_XS grid: 512 x 8 fp16 values
    uint2 *g3h;      // IQ3_XXS grid: 256 x 4 fp16 values
    uint4 *sgn;      // 7-bit sign index -> 8 fp16 sign masks (0x8000 where negative)
    uint32_t *kv2;   // IQ4_XS byte -> {fp16 kvalue[low nibble], fp16 kvalue[high nibble]}
    uint4 *g2sh;     // IQ2_S grid: 1024 x 8 fp16 values
    uint2 *g3sh;     // IQ3_S grid: 512 x 4 fp16 values
    uint4 *sgn8;     // sign byte -> 8 fp16 sign masks (IQ2_S, IQ3_S)
};

// One quantized matrix [rows x K] in the repacked layout (expert e's rows follow e*rows).
struct PfMat {
    const uint8_t *qs, *p1;   // qs plane; IQ4_XS / Q5_K meta, IQ2_XS / IQ2_S scales, IQ3_XXS aux, IQ3_S signs
    const uint8_t *p2;        // Q5_K qh, IQ2_S qh, IQ3_S {qh, scales}
    const uint16_t *d;        // fp16 d per block (IQ2_XS, IQ3_XXS, IQ2_S, IQ3_S)
};

// Arguments of one prefill GEMM launch: Y[row][col] = sum_k A[row][k] * W[col][k], A the
// packed activations (rows = tokens or expert slots), W up to three matrices stacked
// along the output columns (Q, K, V) or, for the expert GEMMs, expert e's slice.
struct PfGemm {
    PfMat w[3];
    uint32_t w_start[3];       // first output column of each stacked matrix
    uint32_t rows;             // rows of one expert's matrix (expert GEMMs)
    uint32_t kb;               // 256-value blocks per matrix row (K / 256)
    const uint4 *apk;          // packed activations
    const float *rscale;       // per packed row: 1/s, 0 for a non-finite row
    const uint32_t *mgroups;   // expert GEMMs: {expert, first m-tile, m-tiles}; null: dense
    const uint32_t *meta;      // expert GEMMs: meta[0] = number of m-groups
    uint32_t mtiles, nvalid;   // dense: m-tiles of 32 rows, valid rows
    float *out;                // output rows of ld floats
    uint32_t ld;
    const float *resid;        // residual added by the O projection epilogue
    float *dump;               // O projection output without the residual (optional)
    uint32_t xcd_rows;         // row-tile classes across the 8 XCDs (1, 2, 4 or 8; the launcher sets it)
};
// GEMM kinds of qxp_launch_gemm (format and epilogue of the weight matrix)
enum QxpGemmKind : int {
    QXP_QKV = 0, QXP_O = 1, QXP_GU = 2, QXP_DOWN = 3,              // the benchmark mix
    QXP_V_Q5 = 4, QXP_O_Q5 = 5, QXP_GU_IQ2S = 6, QXP_DOWN_IQ3S = 7, QXP_DOWN_IQ4 = 8   // real-checkpoint layers
};

// Optional start/stop events recorded around one launch on its stream.  Created with
// hipEventDisableSystemFence, the markers skip the system-scope cache writeback, so
// their elapsed time stays close to the kernel's own duration.
struct Timer {
    hipEvent_t e0 = nullptr, e1 = nullptr;
};

template <typename F, typename... A>
inline void qx_launch(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Timer t, A... args) {
    if (t.e0) (void)hipEventRecord(t.e0, s);
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    if (t.e1) (void)hipEventRecord(t.e1, s);
}

// Phase timestamps for development builds only (-DQXG_TRACE): lane 0 of each wave
// stores s_memrealtime (100 MHz) into qxg_trace_buf[kernel][wave][point]; read back
// with qxg_trace_read.  Normal builds compile the markers out.
#ifdef QXG_TRACE
extern __device__ unsigned long long qxg_trace_buf[8][8192][8];
#define QXG_MARK(kind, point)                                                                  \
    do {                                                                                       \
        const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();                        \
        if ((threadIdx.x & 63) == 0) qxg_trace_buf[kind][blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)][point] = t_; \
    } while (0)
#define QXG_ANCHOR(v) asm volatile("" ::"v"(v))
#else
#define QXG_MARK(kind, point) ((void)0)
#define QXG_ANCHOR(v) ((void)0)
#endif
