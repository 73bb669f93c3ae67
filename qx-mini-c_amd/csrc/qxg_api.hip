// C-ABI implementation of include/qxg.h: context, tensor upload + repack,
// model binding, INT8 KV cache, and the launch sequence of one decode step.
#include "qxg.h"
#include "qxg_internal.h"
#include "qx_grids.h"

#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

extern "C" {
__global__ void qxk_embed(const uint8_t *, uint64_t, const uint32_t *, const DevState *, float *);
__global__ void qxk_attn(const float *, const float *, const float *, Tables, int8_t *, int8_t *, float *, float *,
                         uint32_t, uint32_t, double, const DevState *, float *, float *, float *, double *);
__global__ void qxk_attn_merge(const DevState *, const float *, float *, double *);
__global__ void qxk_stage_route(const double *, uint32_t, float *, DevState *, uint32_t *);
__global__ void qxk_stage_ctx(const float *, uint32_t, float *);
__global__ void qxk_router(const float *, const float *, const float *, uint32_t, double *);
__global__ void qxk_topk(const float *, uint32_t, uint32_t, float *, uint32_t *, float *, uint32_t *, uint32_t *,
                         DevState *);
__global__ void qxk_advance(DevState *, const double *, const double *);
__global__ void qxk_topk_merge(const float *, const uint32_t *, uint32_t, uint32_t, float *, uint32_t *, uint32_t *,
                               DevState *);
__global__ void qxk_q8k(const float *, uint32_t, uint8_t *, uint32_t *);
__global__ void qxk_decode(QxDArgs);
__global__ void qxk_decode_chunked(QxDArgs);
__global__ void qxk_decode_q8(QxDArgs);
__global__ void qxk_decode_chunked_q8(QxDArgs);
__global__ void qxk_interleave_experts(const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *,
                                       const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, uint32_t, uint8_t *,
                                       uint8_t *);
__global__ void qxk_router_fold(const float *, const float *, const float *, uint32_t, float *);
__global__ void qxk_int8_row(const float *, uint32_t, int8_t *, float *);
__global__ void qxk_interleave_head(const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, uint32_t, uint8_t *);
__global__ void qxk_pack_decode(const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *,
                                const uint8_t *, const uint8_t *, const uint8_t *, const float *, const float *, uint32_t,
                                uint8_t *);
__global__ void qxk_dequant(uint32_t, const uint8_t *, const uint8_t *, const uint8_t *, const uint16_t *, Tables,
                            uint64_t, float *);
__global__ void qxk_repack(uint32_t, const uint8_t *, uint64_t, uint8_t *, uint8_t *, uint8_t *, uint16_t *);
void qxl_qkv(hipStream_t, const float *, const float *, const QTensor *, const QTensor *, const QTensor *, float *,
             DevState *, bool, Timer = Timer());
void qxl_oproj(hipStream_t, const float *, const QTensor *, float *, float *, DevState *, bool, Timer = Timer());
void qxl_gate_up(hipStream_t, const float *, const float *, const QTensor *, const QTensor *, Tables, const double *,
                 uint32_t, DevState *, float *, uint32_t *, double *, bool, Timer = Timer(), const uint32_t * = nullptr,
                 float * = nullptr);
void qxl_down(hipStream_t, const float *, const QTensor *, Tables, DevState *, float *, float *, bool,
              Timer = Timer(), float * = nullptr, float * = nullptr);
void qxl_head(hipStream_t, const float *, const float *, const QTensor *, uint32_t, DevState *, float *, float *,
              uint32_t *, bool, Timer = Timer());
__global__ void qxp_embed(const uint8_t *, uint64_t, const uint32_t *, float *);
__global__ void qxp_norm(const float *, const float *, uint32_t, float *);
__global__ void qxp_norm_pack(const float *, const float *, uint32_t, uint32_t, uint4 *, float *);
__global__ void qxp_qk(const float *, const float *, const float *, Tables, int8_t *, int8_t *, float *, float *,
                       uint32_t, uint32_t, uint32_t, float *);
__global__ void qxp_attn(const float *, const int8_t *, const int8_t *, const float *, const float *, uint32_t, uint32_t,
                         uint32_t, uint32_t, float *);
__global__ void qxp_router(const float *, const float *, uint32_t, uint32_t, double *);
__global__ void qxp_route(const double *, uint32_t, uint32_t, uint32_t *, double *);
__global__ void qxp_group(const uint32_t *, uint32_t, uint32_t, uint32_t, int32_t *, uint32_t *, uint32_t *, uint32_t *);
__global__ void qxp_combine(const float *, const float *, const uint32_t *, const double *, float *, float *);
void qxp_launch_gemm(hipStream_t, int, const PfGemm &, const PfTables &, uint32_t, uint32_t, Timer);
void qxp_launch_pack(hipStream_t, int, const float *, const int32_t *, const uint32_t *, uint32_t, uint32_t, uint4 *,
                     float *);
}

namespace {
constexpr uint32_t TOPK_BLOCKS = 128;

void set_err(char *err, uint64_t n, const char *msg) {
    if (err && n) snprintf(err, (size_t)n, "%s", msg);
}

bool hip_ok(hipError_t e, char *err, uint64_t n, const char *what) {
    if (e == hipSuccess) return true;
    if (err && n) snprintf(err, (size_t)n, "%s: %s", what, hipGetErrorString(e));
    return false;
}

uint64_t align256(uint64_t v) { return (v + 255) & ~255ull; }

bool block_geom(uint32_t t, uint64_t &bv, uint64_t &bb) {
    switch (t) {
    case 0: bv = 1; bb = 4; return true;
    case 12: bv = 256; bb = 144; return true;
    case 14: bv = 256; bb = 210; return true;
    case 17: bv = 256; bb = 74; return true;
    case 18: bv = 256; bb = 98; return true;
    case 23: bv = 256; bb = 136; return true;
    case 13: bv = 256; bb = 176; return true;
    case 21: bv = 256; bb = 110; return true;
    case 22: bv = 256; bb = 82; return true;
    default: return false;
    }
}

struct KernelTiming {
    int which = -1;
    std::vector<hipEvent_t> ev;   // pairs
    uint32_t used = 0;
};
}  // namespace

struct qxg_ctx {
    int device = 0;
    hipStream_t s = nullptr;
    Tables T{};
    std::map<std::string, QTensor> tens;
    uint64_t dev_bytes = 0;
    // bound model
    bool bound = false;
    uint32_t layers = 0, vocab = 0, experts = 0;
    std::vector<LayerW> L;
    const uint8_t *emb = nullptr;
    uint64_t emb_row = 0;
    const float *out_norm = nullptr;
    const QTensor *head = nullptr;
    // KV
    int8_t *kc = nullptr, *vc = nullptr;
    float *ks = nullptr, *vs = nullptr;
    uint32_t kv_layers = 0, kv_ctx = 0;
    // work buffers
    float *x = nullptr, *qkv = nullptr, *ctxv = nullptr, *h = nullptr, *logits = nullptr;
    float *vcur = nullptr, *attn = nullptr, *moe = nullptr, *norm = nullptr, *layer_dump = nullptr;
    float *half_dump = nullptr;    // [layer][attention 2048 | MoE 2048] of the last qxg_decode_token step
    double *wsum_dump = nullptr;   // [layer][32] each head's sum of normalised attention weights (same step)
    uint32_t att_split_min = QXD_SPLIT_MIN_DEFAULT;   // persistent decode: chunked stage A from n = pos + 1 on
    double *rlog = nullptr;
    uint32_t *route_ids = nullptr;  // [layer][8] experts of the last step, in rank order
    double *route_w = nullptr;      // [layer][8] their renormalised weights
    float *apart = nullptr;        // per-split attention results [32 heads][QXG_MAX_SPLITS]
    uint32_t att_splits = 1;       // attention splits launched: covers every position the launches reach
    uint32_t graph_splits = 0;     // the recorded step graph's
    float *cand_v = nullptr, *top_v = nullptr;
    uint32_t *cand_i = nullptr, *top_i = nullptr, *tokens = nullptr, *dig = nullptr;
    DevState *st = nullptr;
    uint8_t *staging = nullptr;
    uint64_t staging_bytes = 0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    KernelTiming kt;
    // persistent decode: weight arenas, router fold, tagged exchange buffers, abort flag
    bool persist = true;             // layer path: persistent decode kernel (true, the default) or one kernel per phase
    bool base_mix = true;            // every layer in the benchmark mix (IQ4_XS attention, IQ2_XS/IQ3_XXS experts)
    bool q8 = false;                 // activation mode q8_k_compat (false: f32)
    bool eager = false;              // QXG_EAGER=1 at open: qxg_generate launches every step without a graph
    std::vector<void *> arenas;      // per-plane arenas of all layers' weights
    QxPlane planes[PL_COUNT] = {};
    uint8_t *mfold = nullptr;        // router fold M = W diag(w) O of every layer (f32)
    uint8_t *gu_il = nullptr, *dn_il = nullptr;   // interleaved routed-expert rows of every layer
    uint8_t *head_il = nullptr;                   // interleaved head rows
    uint8_t *dpack = nullptr;                     // decode packs of every layer (QXD_PK_*)
    uint64_t gu_stride = 0, dn_stride = 0;
    uint64_t mfold_stride = 0;
    uint64_t *xch = nullptr;
    uint64_t *xpart = nullptr;       // partial results of the chunked attention (2 x QXD_PART_WORDS)
    uint32_t next_ep = 0;            // epoch base of the next persistent launch
    bool coop_held = false;          // another process holds the GPU's cooperative launches: launch plainly
    uint32_t *abort = nullptr;
    uint8_t *scratch = nullptr;      // device address of this GPU's static workspace (qxg_dequant_blocks_static)
    // one decode step (embed .. head, top-1, step advance) recorded once and replayed
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // batched prefill: codebooks and work buffers for chunks of up to QXP_MAX tokens
    struct Prefill {
        bool ready = false;
        PfTables P{};
        float *X = nullptr, *X1 = nullptr, *XN = nullptr, *QKV = nullptr, *QR = nullptr, *CTX = nullptr;
        float *H = nullptr, *Y = nullptr, *rscale = nullptr, *dump = nullptr;
        uint4 *apk = nullptr;
        double *lg = nullptr, *w = nullptr;
        uint32_t *ids = nullptr, *tok_slot = nullptr, *mgroups = nullptr, *meta = nullptr, *tokens = nullptr;
        int32_t *slot_token = nullptr;
        std::vector<void *> all;
    } pf;
    // stage-probe outputs (allocated on first use)
    struct Stage {
        double *wsum = nullptr;                         // [32] per-head sums of normalised attention weights
        float *norm = nullptr, *route = nullptr;        // [2048] RMSNorm; routing block (2 E + 25 floats)
        float *gu = nullptr, *down = nullptr, *wdown = nullptr;   // [2][8][768] gate, up; [8][2048] down, weighted
        uint32_t *bad = nullptr;
        std::vector<void *> all;
    } sg;
};

namespace {
bool upload_planes(qxg_ctx *c, QTensor &t, const void *host, uint64_t nbytes, char *err, uint64_t n) {
    uint64_t bv = 0, bb = 0;
    block_geom(t.type, bv, bb);
    t.bytes = nbytes;
    t.nblocks = nbytes / bb;
    uint64_t sz[4] = {0, 0, 0, 0};   // p0, p1, p2, d
    const uint64_t nb = t.nblocks;
    switch (t.type) {
    case 23: sz[0] = 128 * nb; sz[1] = 8 * nb; break;
    case 17: sz[0] = 64 * nb; sz[1] = 8 * nb; sz[3] = 2 * nb; break;
    case 18: sz[0] = 64 * nb; sz[1] = 32 * nb; sz[3] = 2 * nb; break;
    case 14: sz[0] = 128 * nb; sz[1] = 64 * nb; sz[2] = 16 * nb; sz[3] = 2 * nb; break;
    case 13: sz[0] = 128 * nb; sz[1] = 16 * nb; sz[2] = 32 * nb; break;
    case 22: sz[0] = 64 * nb; sz[1] = 8 * nb; sz[2] = 8 * nb; sz[3] = 2 * nb; break;
    case 21: sz[0] = 64 * nb; sz[1] = 32 * nb; sz[2] = 16 * nb; sz[3] = 2 * nb; break;
    default: sz[0] = nbytes; break;   // F32, Q4_K: original bytes
    }
    const uint64_t total = align256(sz[0]) + align256(sz[1]) + align256(sz[2]) + align256(sz[3]);
    if (!hip_ok(hipMalloc(&t.base, total), err, n, "hipMalloc tensor")) return false;
    c->dev_bytes += nbytes;
    uint8_t *p = t.base;
    uint8_t *pl[4];
    for (int i = 0; i < 4; ++i) { pl[i] = sz[i] ? p : nullptr; p += align256(sz[i]); }
    t.p0 = pl[0]; t.p1 = pl[1]; t.p2 = pl[2]; t.d = (const uint16_t *)pl[3];
    if (t.type == 0 || t.type == 12) {
        return hip_ok(hipMemcpy(t.base, host, nbytes, hipMemcpyHostToDevice), err, n, "upload");
    }
    if (c->staging_bytes < nbytes) {
        if (c->staging) (void)hipFree(c->staging);
        c->staging = nullptr;
        c->staging_bytes = 0;
        if (!hip_ok(hipMalloc(&c->staging, nbytes), err, n, "hipMalloc staging")) return false;
        c->staging_bytes = nbytes;
    }
    if (!hip_ok(hipMemcpy(c->staging, host, nbytes, hipMemcpyHostToDevice), err, n, "upload")) return false;
    const unsigned grid = (unsigned)((nb + 255) / 256);
    hipLaunchKernelGGL(qxk_repack, dim3(grid), dim3(256), 0, c->s, t.type, c->staging, nb, pl[0], pl[1], pl[2],
                       (uint16_t *)pl[3]);
    if (!hip_ok(hipGetLastError(), err, n, "repack launch")) return false;
    return hip_ok(hipStreamSynchronize(c->s), err, n, "repack");
}

void drop_graph(qxg_ctx *c) {
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->graph_exec = nullptr;
    c->graph = nullptr;
}

void free_tensor(QTensor &t) {
    if (t.base) (void)hipFree(t.base);
    t.base = nullptr;
}

void build_tables_s(std::vector<uint4> &g2s, std::vector<uint2> &g3s, std::vector<uint2> &sel8) {
    g2s.resize(1024);
    for (int i = 0; i < 1024; ++i) {
        uint32_t pos[2] = {0, 0}, neg[2] = {0, 0};
        for (int j = 0; j < 8; ++j) {
            const uint32_t v = qx_iq2xs_levels[(qx_iq2s_packed[i] >> (2 * j)) & 3];
            pos[j >> 2] |= v << (8 * (j & 3));
            neg[j >> 2] |= ((256u - v) & 255u) << (8 * (j & 3));
        }
        g2s[i] = make_uint4(pos[0], pos[1], neg[0], neg[1]);
    }
    g3s.resize(512);
    for (int i = 0; i < 512; ++i) {
        uint32_t pos = 0, neg = 0;
        for (int j = 0; j < 4; ++j) {
            const uint32_t v = qx_iq3s_levels[(qx_iq3s_packed[i] >> (3 * j)) & 7];
            pos |= v << (8 * j);
            neg |= ((256u - v) & 255u) << (8 * j);
        }
        g3s[i] = make_uint2(pos, neg);
    }
    sel8.resize(256);
    for (uint32_t s = 0; s < 256; ++s) {   // explicit sign bytes (IQ2_S, IQ3_S)
        uint32_t a = 0, b = 0;
        for (int j = 0; j < 4; ++j) {
            a |= (uint32_t)(j + 4 * ((s >> j) & 1)) << (8 * j);
            b |= (uint32_t)(j + 4 * ((s >> (j + 4)) & 1)) << (8 * j);
        }
        sel8[s] = make_uint2(a, b);
    }
}

void build_tables(std::vector<uint4> &g2, std::vector<uint2> &g3, std::vector<uint2> &sel) {
    g2.resize(512);
    for (int i = 0; i < 512; ++i) {
        uint32_t pos[2] = {0, 0}, neg[2] = {0, 0};
        for (int j = 0; j < 8; ++j) {
            const uint32_t v = qx_iq2xs_levels[(qx_iq2xs_packed[i] >> (2 * j)) & 3];
            pos[j >> 2] |= v << (8 * (j & 3));
            neg[j >> 2] |= ((256u - v) & 255u) << (8 * (j & 3));
        }
        g2[i] = make_uint4(pos[0], pos[1], neg[0], neg[1]);
    }
    g3.resize(256);
    for (int i = 0; i < 256; ++i) {
        uint32_t pos = 0, neg = 0;
        for (int j = 0; j < 4; ++j) {
            const uint32_t v = qx_iq3xxs_levels[(qx_iq3xxs_packed[i] >> (3 * j)) & 7];
            pos |= v << (8 * j);
            neg |= ((256u - v) & 255u) << (8 * j);
        }
        g3[i] = make_uint2(pos, neg);
    }
    sel.resize(128);
    for (uint32_t i = 0; i < 128; ++i) {
        const uint32_t s = i | ((uint32_t)(__builtin_popcount(i) & 1) << 7);   // ksigns (ggml)
        uint32_t a = 0, b = 0;
        for (int j = 0; j < 4; ++j) {
            a |= (uint32_t)(j + 4 * ((s >> j) & 1)) << (8 * j);
            b |= (uint32_t)(j + 4 * ((s >> (j + 4)) & 1)) << (8 * j);
        }
        sel[i] = make_uint2(a, b);
    }
}

void write_state(qxg_ctx *c, uint32_t pos0, uint32_t step, uint32_t n_prompt, uint32_t force_head) {
    DevState h{};
    h.pos0 = pos0; h.step = step; h.n_prompt = n_prompt; h.force_head = force_head;
    (void)hipMemcpyAsync(c->st, &h, offsetof(DevState, moe_ids), hipMemcpyHostToDevice, c->s);
    // the position's RoPE row, read by the attention kernel without waiting for the position
    const uint64_t p = std::min<uint64_t>((uint64_t)pos0 + step, QXG_MAX_CTX - 1);
    (void)hipMemcpyAsync(c->st->rope_c, c->T.rope_cos + p * 64, 64 * sizeof(double), hipMemcpyDeviceToDevice, c->s);
    (void)hipMemcpyAsync(c->st->rope_s, c->T.rope_sin + p * 64, 64 * sizeof(double), hipMemcpyDeviceToDevice, c->s);
}

const QTensor *find(qxg_ctx *c, const std::string &name) {
    auto it = c->tens.find(name);
    return it == c->tens.end() ? nullptr : &it->second;
}

// Start/stop events for the next launch of kernel `which` while in-situ timing of
// that kernel is enabled; an empty Timer otherwise.
Timer timer_for(qxg_ctx *c, int which) {
    if (c->kt.which != which) return Timer();
    if (c->kt.used * 2 + 2 > c->kt.ev.size()) {
        for (int i = 0; i < 256; ++i) {
            hipEvent_t e;
            (void)hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
            c->kt.ev.push_back(e);
        }
    }
    Timer t;
    t.e0 = c->kt.ev[2 * c->kt.used];
    t.e1 = c->kt.ev[2 * c->kt.used + 1];
    ++c->kt.used;
    return t;
}

// ---- launch sequences (all asynchronous on c->s) ----
void launch_attention(qxg_ctx *c, uint32_t l, float *x, float *attn_dump, float *vcur_dump, double *wsum = nullptr) {
    const LayerW &w = c->L[l];
    qxl_qkv(c->s, x, w.attn_norm, w.wq, w.wk, w.wv, c->qkv, c->st, c->q8, timer_for(c, 2));
    qx_launch(qxk_attn, dim3(32, c->att_splits), dim3(256), 0, c->s, timer_for(c, 5), c->qkv, w.q_norm, w.k_norm,
              c->T, c->kc, c->vc, c->ks, c->vs, l, c->kv_ctx, std::sqrt(128.0), (const DevState *)c->st, c->ctxv,
              c->apart, vcur_dump, wsum);
    if (c->att_splits > 1)
        hipLaunchKernelGGL(qxk_attn_merge, dim3(32), dim3(128), 0, c->s, (const DevState *)c->st, (const float *)c->apart,
                           c->ctxv, wsum);
    qxl_oproj(c->s, c->ctxv, w.wo, x, attn_dump, c->st, c->q8, timer_for(c, 3));
}

void launch_moe(qxg_ctx *c, uint32_t l, float *x, float *moe_dump) {
    const LayerW &w = c->L[l];
    qx_launch(qxk_router, dim3(c->experts), dim3(256), 0, c->s, timer_for(c, 6), (const float *)x,
              w.ffn_norm, w.router, c->experts, c->rlog);
    qxl_gate_up(c->s, x, w.ffn_norm, w.gate, w.up, c->T, c->rlog, c->experts, c->st, c->h, c->route_ids + 8 * l,
                c->route_w + 8 * l, c->q8, timer_for(c, 0));
    qxl_down(c->s, c->h, w.down, c->T, c->st, x, moe_dump, c->q8, timer_for(c, 1));
}

void launch_head(qxg_ctx *c, uint32_t top_n, float *norm_dump) {
    qxl_head(c->s, c->x, c->out_norm, c->head, c->vocab, c->st, c->logits, norm_dump, c->dig, c->q8, timer_for(c, 4));
    hipLaunchKernelGGL(qxk_topk, dim3(TOPK_BLOCKS), dim3(256), 0, c->s, c->logits, c->vocab, top_n, c->cand_v,
                       c->cand_i, c->top_v, c->top_i, c->tokens, c->st);
    hipLaunchKernelGGL(qxk_topk_merge, dim3(1), dim3(256), 0, c->s, (const float *)c->cand_v, (const uint32_t *)c->cand_i,
                       (uint32_t)TOPK_BLOCKS, top_n, c->top_v, c->top_i, c->tokens, c->st);
}

constexpr uint64_t DECODE_WAIT_TICKS = 100000000ull;   // 1 s of the 100 MHz wall clock per wait

// The persistent decode reads the weight arenas and the router fold, built for the
// benchmark mix only (in either activation mode); other models run one kernel per phase.
bool persistent(const qxg_ctx *c) {
    return c->persist && c->base_mix && c->emb && c->head && c->mfold && c->gu_il && c->dn_il && c->head_il && c->dpack;
}

struct DecodeDumps {
    float *layer = nullptr, *res = nullptr, *logits = nullptr, *half = nullptr;
    double *wsum = nullptr;
    float *norm = nullptr;
    uint32_t *rids = nullptr;
    bool rec_all = false;   // every step's dumps, one slot per step of the call
    double *rw = nullptr;
    uint64_t *time = nullptr;   // with rec_all: each step's start and the end, 100 MHz ticks
};

// One cooperative launch of the persistent decode for `steps` steps from pos0 (tokens
// already in c->tokens from index s0: the launch reads tokens[s0 ..] as its own tokens[0 ..]).
// Exchange epochs advance by the launch's phases; before they could wrap, the buffers are
// cleared and the count restarts.
bool launch_decode_part(qxg_ctx *c, bool chunked, uint32_t s0, uint32_t steps, uint32_t n_prompt, uint32_t pos0,
                        bool force_head, const DecodeDumps &d, char *err, uint64_t n) {
    const uint64_t phases = (uint64_t)steps * QXD_PHASES(c->layers) + 1;
    if ((uint64_t)c->next_ep + phases >= 0x7fffffffull) {
        if (!hip_ok(hipMemsetAsync(c->xch, 0, QXD_XCH_WORDS * 8ull, c->s), err, n, "exchange buffers") ||
            !hip_ok(hipMemsetAsync(c->xpart, 0, 2ull * QXD_PART_WORDS * 8, c->s), err, n, "exchange buffers"))
            return false;
        c->next_ep = 0;
    }
    QxDArgs a{};
    for (int i = 0; i < PL_COUNT; ++i) a.P[i] = c->planes[i];
    a.GU = {c->gu_il, c->gu_stride};
    a.DN = {c->dn_il, c->dn_stride};
    a.PK = {c->dpack, (uint64_t)QXG_PBLOCKS * QXD_PK_BYTES};
    a.emb = c->emb; a.emb_row = c->emb_row;
    a.out_norm = c->out_norm;
    a.h_ql = c->head->p0; a.h_qh = c->head->p1; a.h_sc = (const int8_t *)c->head->p2; a.h_d = c->head->d;
    a.h_il = c->head_il;
    a.vocab = c->vocab; a.layers = c->layers; a.experts = c->experts; a.ctx = c->kv_ctx;
    a.steps = steps; a.n_prompt = n_prompt; a.pos0 = pos0; a.force_head = force_head ? 1u : 0u;
    a.tokens = c->tokens + s0;
    a.ep0 = c->next_ep;
    a.T = c->T;
    a.kc = c->kc; a.vc = c->vc; a.ks = c->ks; a.vs = c->vs;
    a.st = c->st;
    a.xch = c->xch;
    a.xpart = c->xpart;
    a.logits = d.logits; a.d_layer = d.layer; a.d_rids = d.rids; a.d_rw = d.rw; a.d_res = d.res; a.d_half = d.half;
    a.d_wsum = d.wsum;
    a.d_norm = d.norm;
    a.rec_all = d.rec_all ? 1u : 0u;
    a.rec_base = s0;
    a.d_time = d.rec_all ? d.time : nullptr;
    a.abort = c->abort;
    a.timeout = DECODE_WAIT_TICKS;
    a.sqrt_hd = std::sqrt(128.0);
    c->next_ep += (uint32_t)phases;
    void *args[] = {&a};
    const Timer t = timer_for(c, 7);
    if (t.e0) (void)hipEventRecord(t.e0, c->s);
    // A cooperative launch fails rather than run unless every workgroup can be resident.  The
    // runtime grants cooperative launches on a GPU to one process at a time: once another
    // process has made one, ours are refused (hipErrorIllegalState) while it lives.  Then the
    // kernel is launched plainly: one workgroup per CU fits (checked at open), so on a GPU not
    // saturated by other work all of them are resident, and every wait is bounded
    // (DECODE_WAIT_TICKS; a timed-out launch exits and the call reports it).
    const void *fn = chunked ? (c->q8 ? (const void *)qxk_decode_chunked_q8 : (const void *)qxk_decode_chunked)
                             : (c->q8 ? (const void *)qxk_decode_q8 : (const void *)qxk_decode);
    hipError_t e = hipErrorIllegalState;
    if (!c->coop_held) {
        e = hipLaunchCooperativeKernel(fn, dim3(QXG_PBLOCKS), dim3(QXD_THREADS), args, 0, c->s);
        if (e == hipErrorIllegalState) {
            (void)hipGetLastError();   // the refusal is not an error of the call
            c->coop_held = true;
        }
    }
    if (c->coop_held) e = hipLaunchKernel(fn, dim3(QXG_PBLOCKS), dim3(QXD_THREADS), args, 0, c->s);
    if (!hip_ok(e, err, n, "persistent decode launch")) return false;
    if (t.e1) (void)hipEventRecord(t.e1, c->s);
    return true;
}

// The persistent decode of steps 0 .. steps-1 at positions pos0 ..: the steps whose cache
// reaches n = pos + 1 >= att_split_min run in the chunked kernel, those before in the walk
// kernel (two launches where the call crosses the threshold; the second reads its first
// token from where the first left it, and its prompt is what remains of the call's).  Each
// launch writes the dumps of its own last step, so the call's last step wins.
bool launch_decode(qxg_ctx *c, uint32_t steps, uint32_t n_prompt, uint32_t pos0, bool force_head,
                   const DecodeDumps &d, char *err, uint64_t n) {
    const uint64_t first_chunked = c->att_split_min > (uint64_t)pos0 + 1 ? (uint64_t)c->att_split_min - 1 - pos0 : 0;
    const uint32_t s1 = (uint32_t)std::min<uint64_t>(first_chunked, steps);
    if (s1 > 0 && !launch_decode_part(c, false, 0, s1, n_prompt, pos0, force_head, d, err, n)) return false;
    if (s1 < steps &&
        !launch_decode_part(c, true, s1, steps - s1, n_prompt > s1 ? n_prompt - s1 : 1u, pos0 + s1, force_head, d, err, n))
        return false;
    return true;
}

// The router fold M = W diag(w) O of every layer (see qxg_decode.hip), from the
// bit-exact dequantized O rows, into one arena (layer l at mfold + l * stride).
bool build_router_fold(qxg_ctx *c, char *err, uint64_t n) {
    if (c->mfold) { (void)hipFree(c->mfold); c->mfold = nullptr; }
    const uint64_t E = c->experts;
    c->mfold_stride = align256(E * 4096 * 4);
    float *o = nullptr;
    if (!hip_ok(hipMalloc(&c->mfold, c->mfold_stride * c->layers), err, n, "router fold") ||
        !hip_ok(hipMalloc(&o, 2048ull * 4096 * 4), err, n, "router fold"))
        return false;
    bool ok = true;
    for (uint32_t l = 0; l < c->layers && ok; ++l) {
        const LayerW &w = c->L[l];
        const uint64_t nb = w.wo->nblocks;   // 2048 rows x 16 blocks
        hipLaunchKernelGGL(qxk_dequant, dim3((unsigned)nb), dim3(256), 0, c->s, 23u, w.wo->p0, w.wo->p1, w.wo->p2, w.wo->d,
                           c->T, nb, o);
        hipLaunchKernelGGL(qxk_router_fold, dim3(16, (unsigned)((E + 3) / 4)), dim3(256), 0, c->s, w.router, w.ffn_norm,
                           (const float *)o, (uint32_t)E, (float *)(c->mfold + l * c->mfold_stride));
        ok = hip_ok(hipGetLastError(), err, n, "router fold");
    }
    ok = ok && hip_ok(hipStreamSynchronize(c->s), err, n, "router fold");
    (void)hipFree(o);
    return ok;
}

// The routed experts' rows of every layer in the persistent decode's interleaved layout
// (QXD_GU_UNIT, QXD_DN_ROW in qxg_internal.h), copied from the IQ2_XS / IQ3_XXS planes.
bool build_expert_interleave(qxg_ctx *c, char *err, uint64_t n) {
    for (uint8_t **p : {&c->gu_il, &c->dn_il})
        if (*p) { (void)hipFree(*p); *p = nullptr; }
    const uint64_t E = c->experts;
    c->gu_stride = align256(E * 768 * QXD_GU_UNIT);
    c->dn_stride = align256(E * 2048 * QXD_DN_ROW);
    if (!hip_ok(hipMalloc(&c->gu_il, c->gu_stride * c->layers), err, n, "expert interleave") ||
        !hip_ok(hipMalloc(&c->dn_il, c->dn_stride * c->layers), err, n, "expert interleave"))
        return false;
    bool ok = true;
    const unsigned grid = (unsigned)((E * (768 + 2048) + 255) / 256);
    for (uint32_t l = 0; l < c->layers && ok; ++l) {
        const LayerW &w = c->L[l];
        hipLaunchKernelGGL(qxk_interleave_experts, dim3(grid), dim3(256), 0, c->s, w.gate->p0, w.gate->p1, (const uint8_t *)w.gate->d,
                           w.up->p0, w.up->p1, (const uint8_t *)w.up->d, w.down->p0, w.down->p1, (const uint8_t *)w.down->d,
                           (uint32_t)E, c->gu_il + l * c->gu_stride, c->dn_il + l * c->dn_stride);
        ok = hip_ok(hipGetLastError(), err, n, "expert interleave");
    }
    if (ok && c->head) {
        if (c->head_il) { (void)hipFree(c->head_il); c->head_il = nullptr; }
        ok = hip_ok(hipMalloc(&c->head_il, (uint64_t)c->vocab * QXD_HEAD_ROW), err, n, "head interleave");
        if (ok) {
            hipLaunchKernelGGL(qxk_interleave_head, dim3((c->vocab + 255) / 256), dim3(256), 0, c->s, c->head->p0, c->head->p1,
                               c->head->p2, (const uint8_t *)c->head->d, c->vocab, c->head_il);
            ok = hip_ok(hipGetLastError(), err, n, "head interleave");
        }
    }
    return ok && hip_ok(hipStreamSynchronize(c->s), err, n, "expert interleave");
}

// The persistent decode's packs (QXD_PK_* in qxg_internal.h): per layer, each workgroup's
// Q/K/V/O rows with their metas, router row and router-fold row, contiguous.  After the
// arenas and the router fold.
bool build_decode_pack(qxg_ctx *c, char *err, uint64_t n) {
    if (c->dpack) { (void)hipFree(c->dpack); c->dpack = nullptr; }
    if (c->experts < 1 || c->experts > QXG_PBLOCKS || !c->mfold) return true;   // no persistent decode for this model
    const uint64_t stride = (uint64_t)QXG_PBLOCKS * QXD_PK_BYTES;
    if (!hip_ok(hipMalloc(&c->dpack, stride * c->layers), err, n, "decode pack")) return false;
    bool ok = true;
    for (uint32_t l = 0; l < c->layers && ok; ++l) {
        const LayerW &w = c->L[l];
        hipLaunchKernelGGL(qxk_pack_decode, dim3(QXG_PBLOCKS), dim3(256), 0, c->s, w.wq->p0, w.wq->p1, w.wk->p0, w.wk->p1,
                           w.wv->p0, w.wv->p1, w.wo->p0, w.wo->p1, w.router,
                           (const float *)(c->mfold + l * c->mfold_stride), (uint32_t)c->experts, c->dpack + l * stride);
        ok = hip_ok(hipGetLastError(), err, n, "decode pack");
    }
    return ok && hip_ok(hipStreamSynchronize(c->s), err, n, "decode pack");
}

void launch_step(qxg_ctx *c, uint32_t top_n, bool dump_layers) {
    hipLaunchKernelGGL(qxk_embed, dim3(1), dim3(256), 0, c->s, c->emb, c->emb_row, c->tokens, c->st, c->x);
    for (uint32_t l = 0; l < c->layers; ++l) {
        launch_attention(c, l, c->x, nullptr, nullptr);
        launch_moe(c, l, c->x, nullptr);
        if (dump_layers)
            (void)hipMemcpyAsync(c->layer_dump + 2048ull * l, c->x, 2048 * sizeof(float), hipMemcpyDeviceToDevice, c->s);
    }
    if (c->head) launch_head(c, top_n, nullptr);
}

// A persistent launch whose waits timed out leaves the abort flag set: report and clear it.
bool check_abort(qxg_ctx *c, char *err, uint64_t n) {
    uint32_t f = 0;
    if (!hip_ok(hipMemcpy(&f, c->abort, 4, hipMemcpyDeviceToHost), err, n, "abort flag")) return false;
    if (!f) return true;
    (void)hipMemset(c->abort, 0, 4);
    set_err(err, n, "persistent decode: a wait timed out (a workgroup never produced its phase output)");
    return false;
}

bool check_ready(qxg_ctx *c, bool need_kv, char *err, uint64_t n) {
    if (!c) { set_err(err, n, "invalid context"); return false; }
    if (!c->bound) { set_err(err, n, "model not bound"); return false; }
    if (need_kv && !c->kc) { set_err(err, n, "KV cache not created"); return false; }
    return true;
}

// A q8_k_compat step that met a non-finite activation or expert row leaves a fault code
// in the state: report it with the reference's message and clear it.
bool check_q8(qxg_ctx *c, char *err, uint64_t n) {
    uint32_t f = 0;
    if (!hip_ok(hipMemcpy(&f, &c->st->q8_fault, 4, hipMemcpyDeviceToHost), err, n, "state read")) return false;
    if (!f) return true;
    (void)hipMemset(&c->st->q8_fault, 0, 4);
    set_err(err, n, f == QXG_Q8_NONFINITE_EXPERT ? "non-finite packed expert Q8_K output" : "Q8_K activation contains NaN or Inf");
    return false;
}

bool finish(qxg_ctx *c, char *err, uint64_t n) {
    if (!hip_ok(hipGetLastError(), err, n, "launch")) return false;
    if (!hip_ok(hipStreamSynchronize(c->s), err, n, "stream")) return false;
    if (c->q8 && !check_q8(c, err, n)) return false;
    return !c->abort || check_abort(c, err, n);
}

bool read_state(qxg_ctx *c, DevState &h, char *err, uint64_t n) {
    return hip_ok(hipMemcpyAsync(&h, c->st, sizeof(h), hipMemcpyDeviceToHost, c->s), err, n, "state read") &&
           hip_ok(hipStreamSynchronize(c->s), err, n, "stream");
}
// Every per-layer weight plane (norms, router, the quantized planes of Q/K/V/O and
// of the expert tensors) is copied into one arena per plane kind, layers back to
// back at a 256-byte-aligned stride; the tensors are re-pointed into the arenas and
// their own allocations released.  The decode kernel then forms layer l's pointers
// as base + l * stride from its arguments.
bool build_arenas(qxg_ctx *c, char *err, uint64_t n) {
    const uint32_t L = c->layers ? c->layers : (uint32_t)c->L.size();
    std::vector<void *> old = std::move(c->arenas);
    c->arenas.clear();
    struct Src { const uint8_t *p; uint64_t bytes; };
    auto src = [&](int id, uint32_t l) -> Src {
        const LayerW &w = c->L[l];
        const uint64_t E = c->experts;
        switch (id) {
        case PL_ATTN_NORM: return {(const uint8_t *)w.attn_norm, 2048 * 4};
        case PL_Q_NORM: return {(const uint8_t *)w.q_norm, 128 * 4};
        case PL_K_NORM: return {(const uint8_t *)w.k_norm, 128 * 4};
        case PL_FFN_NORM: return {(const uint8_t *)w.ffn_norm, 2048 * 4};
        case PL_ROUTER: return {(const uint8_t *)w.router, E * 2048 * 4};
        case PL_Q_QS: return {w.wq->p0, w.wq->nblocks * 128};
        case PL_Q_META: return {w.wq->p1, w.wq->nblocks * 8};
        case PL_K_QS: return {w.wk->p0, w.wk->nblocks * 128};
        case PL_K_META: return {w.wk->p1, w.wk->nblocks * 8};
        case PL_V_QS: return {w.wv->p0, w.wv->nblocks * 128};
        case PL_V_META: return {w.wv->p1, w.wv->nblocks * 8};
        case PL_O_QS: return {w.wo->p0, w.wo->nblocks * 128};
        case PL_O_META: return {w.wo->p1, w.wo->nblocks * 8};
        case PL_G_QS: return {w.gate->p0, w.gate->nblocks * 64};
        case PL_G_SC: return {w.gate->p1, w.gate->nblocks * 8};
        case PL_G_D: return {(const uint8_t *)w.gate->d, w.gate->nblocks * 2};
        case PL_U_QS: return {w.up->p0, w.up->nblocks * 64};
        case PL_U_SC: return {w.up->p1, w.up->nblocks * 8};
        case PL_U_D: return {(const uint8_t *)w.up->d, w.up->nblocks * 2};
        case PL_D_QS: return {w.down->p0, w.down->nblocks * 64};
        case PL_D_AUX: return {w.down->p1, w.down->nblocks * 32};
        default: return {(const uint8_t *)w.down->d, w.down->nblocks * 2};
        }
    };
    // the four norm vectors of a layer together (QXD_NORM_STRIDE): one translation page
    // holds every layer's
    uint8_t *norms = nullptr;
    if (!hip_ok(hipMalloc(&norms, (uint64_t)QXD_NORM_STRIDE * L), err, n, "weight arena")) return false;
    c->arenas.push_back(norms);
    const uint64_t norm_off[4] = {0, 16384, 16896, 8192};   // PL_ATTN_NORM, PL_Q_NORM, PL_K_NORM, PL_FFN_NORM
    static_assert(PL_ATTN_NORM == 0 && PL_Q_NORM == 1 && PL_K_NORM == 2 && PL_FFN_NORM == 3, "norm planes first");
    for (int id = 0; id < PL_COUNT; ++id) {
        uint8_t *ar = nullptr;
        uint64_t stride;
        if (id <= PL_FFN_NORM) {
            ar = norms + norm_off[id];
            stride = QXD_NORM_STRIDE;
        } else {
            stride = align256(src(id, 0).bytes);
            if (!hip_ok(hipMalloc(&ar, stride * L), err, n, "weight arena")) return false;
            c->arenas.push_back(ar);
        }
        for (uint32_t l = 0; l < L; ++l) {
            const Src sp = src(id, l);
            if (!hip_ok(hipMemcpyAsync(ar + l * stride, sp.p, sp.bytes, hipMemcpyDeviceToDevice, c->s), err, n, "weight arena"))
                return false;
        }
        c->planes[id] = {ar, stride};
    }
    if (!hip_ok(hipStreamSynchronize(c->s), err, n, "weight arena")) return false;
    auto at = [&](int id, uint32_t l) { return c->planes[id].base + (uint64_t)l * c->planes[id].stride; };
    for (uint32_t l = 0; l < L; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        struct { const char *sfx; int p0, p1, d; } q[] = {
            {"attn_q.weight", PL_Q_QS, PL_Q_META, -1}, {"attn_k.weight", PL_K_QS, PL_K_META, -1},
            {"attn_v.weight", PL_V_QS, PL_V_META, -1}, {"attn_output.weight", PL_O_QS, PL_O_META, -1},
            {"ffn_gate_exps.weight", PL_G_QS, PL_G_SC, PL_G_D}, {"ffn_up_exps.weight", PL_U_QS, PL_U_SC, PL_U_D},
            {"ffn_down_exps.weight", PL_D_QS, PL_D_AUX, PL_D_D}, {"attn_norm.weight", PL_ATTN_NORM, -1, -1},
            {"attn_q_norm.weight", PL_Q_NORM, -1, -1}, {"attn_k_norm.weight", PL_K_NORM, -1, -1},
            {"ffn_norm.weight", PL_FFN_NORM, -1, -1}, {"ffn_gate_inp.weight", PL_ROUTER, -1, -1}};
        for (auto &e : q) {
            QTensor &t = c->tens[p + e.sfx];
            free_tensor(t);
            t.p0 = at(e.p0, l);
            t.p1 = e.p1 >= 0 ? at(e.p1, l) : nullptr;
            t.p2 = nullptr;
            t.d = e.d >= 0 ? (const uint16_t *)at(e.d, l) : nullptr;
        }
        LayerW &w = c->L[l];
        w.attn_norm = (const float *)at(PL_ATTN_NORM, l);
        w.q_norm = (const float *)at(PL_Q_NORM, l);
        w.k_norm = (const float *)at(PL_K_NORM, l);
        w.ffn_norm = (const float *)at(PL_FFN_NORM, l);
        w.router = (const float *)at(PL_ROUTER, l);
    }
    for (void *pp : old) (void)hipFree(pp);
    return true;
}

// ---- batched prefill
constexpr uint32_t PF_EXPERT_MT = QXG_PF_EXPERT_MT;               // row tiles per expert GEMM wave
constexpr uint32_t PF_SLOTS = QXP_MAX * QXG_TOPK + 32 * 128;       // expert slots, padded per expert
constexpr uint32_t PF_MGROUPS = QXP_MAX * QXG_TOPK / 32 + 128;     // bound on expert m-groups

// fp16 bits of a small integer (|v| < 2048: exact)
uint16_t f16_int(int v) {
    if (v == 0) return 0;
    const uint16_t sign = v < 0 ? 0x8000 : 0;
    uint32_t a = (uint32_t)(v < 0 ? -v : v);
    int e = 31 - __builtin_clz(a);
    const uint32_t mant = (a << (10 - e)) & 0x3ffu;
    return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | mant);
}

// The batched GEMM path takes every bound format in the f32 activation mode; q8_k_compat
// prefills token by token through the decode kernels, which is how the reference
// prefills every prompt.
bool batched_prefill(const qxg_ctx *c) { return !c->q8; }

bool prefill_ready(qxg_ctx *c, char *err, uint64_t n) {
    auto &B = c->pf;
    if (B.ready) return true;
    auto alloc = [&](void **p, uint64_t bytes) {
        if (!hip_ok(hipMalloc(p, bytes), err, n, "prefill buffers")) return false;
        B.all.push_back(*p);
        return true;
    };
    const uint64_t T = QXP_MAX;
    bool ok = alloc((void **)&B.X, T * 2048 * 4) && alloc((void **)&B.X1, T * 2048 * 4) &&
              alloc((void **)&B.XN, T * 2048 * 4) && alloc((void **)&B.QKV, T * 5120 * 4) &&
              alloc((void **)&B.QR, T * 4096 * 4) && alloc((void **)&B.CTX, T * 4096 * 4) &&
              alloc((void **)&B.H, (uint64_t)PF_SLOTS * QXG_FFN * 4) && alloc((void **)&B.Y, (uint64_t)PF_SLOTS * 2048 * 4) &&
              alloc((void **)&B.rscale, (uint64_t)PF_SLOTS * 4) && alloc((void **)&B.dump, T * 2048 * 4) &&
              alloc((void **)&B.apk, (uint64_t)PF_SLOTS * 2048 * 4) && alloc((void **)&B.lg, T * 128 * 8) &&
              alloc((void **)&B.w, T * 8 * 8) && alloc((void **)&B.ids, T * 8 * 4) && alloc((void **)&B.tok_slot, T * 8 * 4) &&
              alloc((void **)&B.mgroups, PF_MGROUPS * 4) && alloc((void **)&B.meta, 16) && alloc((void **)&B.tokens, T * 4) &&
              alloc((void **)&B.slot_token, (uint64_t)PF_SLOTS * 4);
    // codebooks: IQ2_XS / IQ3_XXS grids and the IQ4_XS byte table as fp16, sign masks
    std::vector<uint16_t> g2(512 * 8), g3(256 * 4), sg(128 * 8);
    std::vector<uint32_t> kv2(256);
    for (int i = 0; i < 512; ++i)
        for (int j = 0; j < 8; ++j) g2[i * 8 + j] = f16_int(qx_iq2xs_levels[(qx_iq2xs_packed[i] >> (2 * j)) & 3]);
    for (int i = 0; i < 256; ++i)
        for (int j = 0; j < 4; ++j) g3[i * 4 + j] = f16_int(qx_iq3xxs_levels[(qx_iq3xxs_packed[i] >> (3 * j)) & 7]);
    for (uint32_t i = 0; i < 128; ++i) {
        const uint32_t sbits = i | ((uint32_t)(__builtin_popcount(i) & 1) << 7);   // ksigns (ggml)
        for (int j = 0; j < 8; ++j) sg[i * 8 + j] = ((sbits >> j) & 1) ? 0x8000 : 0;
    }
    for (uint32_t b = 0; b < 256; ++b)
        kv2[b] = (uint32_t)f16_int(qx_iq4nl_values[b & 15]) | ((uint32_t)f16_int(qx_iq4nl_values[b >> 4]) << 16);
    // the real checkpoint's IQ2_S / IQ3_S grids as fp16, and sign masks of an explicit sign byte
    std::vector<uint16_t> g2s(1024 * 8), g3s(512 * 4), sg8(256 * 8);
    for (int i = 0; i < 1024; ++i)
        for (int j = 0; j < 8; ++j) g2s[i * 8 + j] = f16_int(qx_iq2xs_levels[(qx_iq2s_packed[i] >> (2 * j)) & 3]);
    for (int i = 0; i < 512; ++i)
        for (int j = 0; j < 4; ++j) g3s[i * 4 + j] = f16_int(qx_iq3s_levels[(qx_iq3s_packed[i] >> (3 * j)) & 7]);
    for (uint32_t i = 0; i < 256; ++i)
        for (int j = 0; j < 8; ++j) sg8[i * 8 + j] = ((i >> j) & 1) ? 0x8000 : 0;
    ok = ok && alloc((void **)&B.P.g2h, g2.size() * 2) && alloc((void **)&B.P.g3h, g3.size() * 2) &&
         alloc((void **)&B.P.sgn, sg.size() * 2) && alloc((void **)&B.P.kv2, kv2.size() * 4) &&
         alloc((void **)&B.P.g2sh, g2s.size() * 2) && alloc((void **)&B.P.g3sh, g3s.size() * 2) &&
         alloc((void **)&B.P.sgn8, sg8.size() * 2);
    ok = ok && hip_ok(hipMemcpy(B.P.g2h, g2.data(), g2.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.g3h, g3.data(), g3.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.sgn, sg.data(), sg.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.kv2, kv2.data(), kv2.size() * 4, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.g2sh, g2s.data(), g2s.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.g3sh, g3s.data(), g3s.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables") &&
         hip_ok(hipMemcpy(B.P.sgn8, sg8.data(), sg8.size() * 2, hipMemcpyHostToDevice), err, n, "prefill tables");
    if (!ok) {
        for (void *p : B.all) (void)hipFree(p);
        B.all.clear();
        return false;
    }
    B.ready = true;
    return true;
}

PfMat pf_mat(const QTensor *t) { return PfMat{t->p0, t->p1, t->p2, t->d}; }

// One layer over the T tokens of a chunk at positions p0..p0+T-1: pf.X -> pf.X (pf.X1
// holds the attention half's result, the MoE input).  Asynchronous on c->s.
void prefill_layer(qxg_ctx *c, uint32_t l, uint32_t T, uint32_t p0, float *moe_dump) {
    auto &B = c->pf;
    const LayerW &w = c->L[l];
    hipStream_t s = c->s;
    const uint32_t mt = (T + 31) / 32, E = c->experts;
    const uint32_t none = 0xffffffffu;
    // attention half: RMSNorm, Q/K/V GEMM, q/k norm + RoPE + INT8 append, attention, O GEMM + residual
    hipLaunchKernelGGL(qxp_norm_pack, dim3(mt * 8), dim3(256), 0, s, (const float *)B.X, w.attn_norm, mt * 32, T, B.apk,
                       B.rscale);
    // per-layer formats of the real checkpoint: V and O in Q5_K or IQ4_XS, gate/up in IQ2_S or
    // IQ2_XS, down in IQ3_XXS, IQ3_S or IQ4_XS (type ids of the QXF1 manifest)
    const bool vo_q5 = w.wv->type == 13, gu_s = w.gate->type == 22;
    const int dn_kind = w.down->type == 21 ? QXP_DOWN_IQ3S : w.down->type == 23 ? QXP_DOWN_IQ4 : QXP_DOWN;
    PfGemm g{};
    g.w[0] = pf_mat(w.wq); g.w[1] = pf_mat(w.wk); g.w[2] = pf_mat(w.wv);
    g.w_start[0] = 0; g.w_start[1] = 4096; g.w_start[2] = vo_q5 ? none : 4608;
    g.kb = 8; g.apk = B.apk; g.rscale = B.rscale; g.mtiles = mt; g.nvalid = T; g.out = B.QKV; g.ld = 5120;
    qxp_launch_gemm(s, QXP_QKV, g, B.P, (vo_q5 ? 4608 : 5120) / 128, mt, timer_for(c, 8));
    if (vo_q5) {   // V (Q5_K) into columns 4608..5119
        PfGemm gv = g;
        gv.w[0] = pf_mat(w.wv); gv.w_start[1] = none; gv.w_start[2] = none; gv.out = B.QKV + 4608;
        qxp_launch_gemm(s, QXP_V_Q5, gv, B.P, 512 / 128, mt, Timer{});
    }
    hipLaunchKernelGGL(qxp_qk, dim3(T), dim3(256), 0, s, (const float *)B.QKV, w.q_norm, w.k_norm, c->T, c->kc, c->vc,
                       c->ks, c->vs, l, c->kv_ctx, p0, B.QR);
    qx_launch(qxp_attn, dim3(4, (T + 3) / 4), dim3(256), 0, s, timer_for(c, 13), (const float *)B.QR,
              (const int8_t *)c->kc, (const int8_t *)c->vc, (const float *)c->ks, (const float *)c->vs, l, c->kv_ctx, p0, T,
              B.CTX);
    qxp_launch_pack(s, 4096, B.CTX, nullptr, nullptr, mt * 32, T, B.apk, B.rscale);
    g = PfGemm{};
    g.w[0] = pf_mat(w.wo); g.w_start[1] = none; g.w_start[2] = none;
    g.kb = 16; g.apk = B.apk; g.rscale = B.rscale; g.mtiles = mt; g.nvalid = T; g.out = B.X1; g.ld = 2048;
    g.resid = B.X;
    qxp_launch_gemm(s, vo_q5 ? QXP_O_Q5 : QXP_O, g, B.P, 2048 / 128, mt, timer_for(c, 9));
    // MoE half: RMSNorm, router logits, top-8, grouping by expert, gate/up + SwiGLU, down, combine
    hipLaunchKernelGGL(qxp_norm, dim3((T + 3) / 4), dim3(256), 0, s, (const float *)B.X1, w.ffn_norm, T, B.XN);
    qx_launch(qxp_router, dim3((T + 15) / 16, (E + 15) / 16), dim3(512), 0, s, timer_for(c, 12), (const float *)B.XN,
              w.router, T, E, B.lg);
    hipLaunchKernelGGL(qxp_route, dim3((T + 3) / 4), dim3(256), 0, s, (const double *)B.lg, T, E, B.ids, B.w);
    hipLaunchKernelGGL(qxp_group, dim3(1), dim3(1024), 0, s, (const uint32_t *)B.ids, T, E, PF_EXPERT_MT, B.slot_token,
                       B.tok_slot, B.mgroups, B.meta);
    const uint32_t slots_ub = T * QXG_TOPK + 32 * E;        // padded slots never exceed this
    const uint32_t mg_ub = (T * QXG_TOPK + 31) / 32 + E;      // nor the m-groups this
    qxp_launch_pack(s, 2048, B.XN, B.slot_token, B.meta, slots_ub, none, B.apk, B.rscale);
    g = PfGemm{};
    g.w[0] = pf_mat(w.gate); g.w[1] = pf_mat(w.up); g.w_start[1] = none; g.w_start[2] = none;
    g.rows = QXG_FFN; g.kb = 8; g.apk = B.apk; g.rscale = B.rscale; g.mgroups = B.mgroups; g.meta = B.meta;
    g.out = B.H; g.ld = QXG_FFN;
    qxp_launch_gemm(s, gu_s ? QXP_GU_IQ2S : QXP_GU, g, B.P, QXG_FFN / 128, mg_ub, timer_for(c, 10));
    qxp_launch_pack(s, 768, B.H, nullptr, B.meta, slots_ub, none, B.apk, B.rscale);
    g = PfGemm{};
    g.w[0] = pf_mat(w.down); g.w_start[1] = none; g.w_start[2] = none;
    g.rows = 2048; g.kb = 3; g.apk = B.apk; g.rscale = B.rscale; g.mgroups = B.mgroups; g.meta = B.meta;
    g.out = B.Y; g.ld = 2048;
    qxp_launch_gemm(s, dn_kind, g, B.P, 2048 / 128, mg_ub, timer_for(c, 11));
    hipLaunchKernelGGL(qxp_combine, dim3(T), dim3(256), 0, s, (const float *)B.X1, (const float *)B.Y,
                       (const uint32_t *)B.tok_slot, (const double *)B.w, B.X, moe_dump);
}
// Token-step prefill: one decode step per prompt token (embedding, every layer), the head
// on the last when run_head; residual_out row i is token i's final residual.
int prefill_steps(qxg_ctx *c, const uint32_t *tokens, uint32_t n, uint32_t position0, int run_head,
                  float *residual_out, uint32_t top_n, char *err, uint64_t err_len) {
    if (!hip_ok(hipMemcpy(c->tokens, tokens, 4ull * n, hipMemcpyHostToDevice), err, err_len, "tokens")) return 0;
    (void)hipEventRecord(c->e0, c->s);
    for (uint32_t i = 0; i < n; ++i) {
        write_state(c, position0, i, run_head ? n : n + 1, 0);   // steps before n_prompt - 1 skip the head
        hipLaunchKernelGGL(qxk_embed, dim3(1), dim3(256), 0, c->s, c->emb, c->emb_row, c->tokens, c->st, c->x);
        for (uint32_t l = 0; l < c->layers; ++l) {
            launch_attention(c, l, c->x, nullptr, nullptr);
            launch_moe(c, l, c->x, nullptr);
        }
        if (residual_out &&
            !hip_ok(hipMemcpyAsync(residual_out + 2048ull * i, c->x, 2048 * 4, hipMemcpyDeviceToHost, c->s), err, err_len, "read"))
            return 0;
        if (i + 1 == n && run_head) launch_head(c, top_n, nullptr);
    }
    (void)hipEventRecord(c->e1, c->s);
    return 1;
}

// Waits for the prefill's work and reads the head's outputs of the last token.
int prefill_finish(qxg_ctx *c, int run_head, float *logits, uint32_t top_n, uint32_t *top_ids, double *top_logits,
                   float *elapsed_ms, char *err, uint64_t err_len) {
    if (!finish(c, err, err_len)) return 0;
    if (elapsed_ms) (void)hipEventElapsedTime(elapsed_ms, c->e0, c->e1);
    if (!run_head) return 1;
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (logits && !hip_ok(hipMemcpy(logits, c->logits, (uint64_t)c->vocab * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    float tv[QXG_MAX_TOPN];
    uint32_t ti[QXG_MAX_TOPN];
    if (!hip_ok(hipMemcpy(tv, c->top_v, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read") ||
        !hip_ok(hipMemcpy(ti, c->top_i, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    for (uint32_t i = 0; i < top_n; ++i) {
        if (top_ids) top_ids[i] = ti[i];
        if (top_logits) top_logits[i] = (double)tv[i];
    }
    if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
    return 1;
}

}  // namespace

// ---- the static workspace of qxg_dequant_blocks_static ----
// The repacked block planes of an allocation-free dequant live in `scratch`, a file-scope
// device array: each GPU the library runs on holds its own copy until the process ends.
// On the host the array's name is only a stand-in for it, so host code never passes it
// on: qxg_open looks up its device address once per device, with that device current
// (hipGetSymbolAddress), and every kernel argument uses that address.  Layout for
// QXG_STATIC_MAX_BLOCKS blocks: planes p0 (128 bytes per block), p1 (64), p2 (32) and
// d (2) back to back - the largest of each over the supported block types.
constexpr uint64_t SCR_P0 = 0, SCR_P1 = 128ull * QXG_STATIC_MAX_BLOCKS, SCR_P2 = 192ull * QXG_STATIC_MAX_BLOCKS,
                   SCR_D = 224ull * QXG_STATIC_MAX_BLOCKS, SCR_BYTES = 226ull * QXG_STATIC_MAX_BLOCKS;
static __device__ __align__(256) uint8_t scratch[SCR_BYTES];

namespace {
std::mutex g_scratch_mu;
std::map<int, uint8_t *> g_scratch_addr;   // device -> address of its copy of `scratch`
std::map<int, std::mutex> g_scratch_use;   // device -> held by a call using its copy (repack through finish)

std::mutex &scratch_use(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_use[device];   // (map nodes do not move)
}

// the calling thread's current device must be `device`
bool scratch_address(int device, uint8_t **addr, char *err, uint64_t n) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_addr.find(device);
    if (it == g_scratch_addr.end()) {
        void *p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), err, n, "hipGetSymbolAddress(scratch)")) return false;
        it = g_scratch_addr.emplace(device, (uint8_t *)p).first;
    }
    *addr = it->second;
    return true;
}
}  // namespace

extern "C" {

int qxg_open(int device, qxg_ctx **out, char *err, uint64_t err_len) {
    if (!out) { set_err(err, err_len, "invalid argument"); return 0; }
    *out = nullptr;
    int count = 0;
    if (!hip_ok(hipGetDeviceCount(&count), err, err_len, "hipGetDeviceCount")) return 0;
    if (device < 0 || device >= count) { set_err(err, err_len, "no such HIP device"); return 0; }
    if (!hip_ok(hipSetDevice(device), err, err_len, "hipSetDevice")) return 0;
    hipDeviceProp_t prop;
    if (!hip_ok(hipGetDeviceProperties(&prop, device), err, err_len, "hipGetDeviceProperties")) return 0;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (err && err_len) snprintf(err, (size_t)err_len, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
        return 0;
    }
    {   // the persistent decode keeps one workgroup resident on each of QXG_PBLOCKS CUs (a
        // cooperative launch where the runtime grants one, see launch_decode_part)
        int occ = 0, coop = 0;
        if (prop.multiProcessorCount < QXG_PBLOCKS ||
            hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess || !coop ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)qxk_decode, QXD_THREADS, 0) != hipSuccess || occ < 1 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)qxk_decode_chunked, QXD_THREADS, 0) != hipSuccess || occ < 1 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)qxk_decode_q8, QXD_THREADS, 0) != hipSuccess || occ < 1 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)qxk_decode_chunked_q8, QXD_THREADS, 0) != hipSuccess || occ < 1) {
            if (err && err_len)
                snprintf(err, (size_t)err_len, "device %d has %d CUs; the persistent decode kernel needs %d resident workgroups",
                         device, prop.multiProcessorCount, QXG_PBLOCKS);
            return 0;
        }
    }
    uint8_t *scr = nullptr;
    if (!scratch_address(device, &scr, err, err_len)) return 0;
    qxg_ctx *c = new qxg_ctx();
    c->device = device;
    c->scratch = scr;
    {
        const char *ev = getenv("QXG_EAGER");
        c->eager = ev && ev[0] == '1';
    }
    bool ok = hip_ok(hipStreamCreateWithFlags(&c->s, hipStreamNonBlocking), err, err_len, "stream");
    std::vector<uint4> g2, g2s;
    std::vector<uint2> g3, sel, g3s, sel8;
    build_tables(g2, g3, sel);
    build_tables_s(g2s, g3s, sel8);
    std::vector<double> rc((size_t)QXG_MAX_CTX * 64), rs((size_t)QXG_MAX_CTX * 64);
    // reference qx_apply_rope (src/qx_format.c:4625-4641): f = pow(theta, -(2i)/hd), angle = pos*f,
    // double cos/sin -- evaluated once here with the host libm.
    for (uint32_t p = 0; p < QXG_MAX_CTX; ++p)
        for (uint32_t i = 0; i < 64; ++i) {
            const double f = pow(1000000.0, -(2.0 * (double)i) / 128.0);
            const double a = (double)p * f;
            rc[p * 64 + i] = cos(a);
            rs[p * 64 + i] = sin(a);
        }
    std::vector<double> rcs((size_t)QXG_MAX_CTX * 128);   // per position: 64 cos, then 64 sin (one page)
    for (uint32_t p = 0; p < QXG_MAX_CTX; ++p)
        for (uint32_t i = 0; i < 64; ++i) {
            rcs[p * 128 + i] = rc[p * 64 + i];
            rcs[p * 128 + 64 + i] = rs[p * 64 + i];
        }
    ok = ok && hip_ok(hipMalloc(&c->T.g2, g2.size() * sizeof(uint4)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.g3, g3.size() * sizeof(uint2)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.sel, sel.size() * sizeof(uint2)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.rope_cos, rc.size() * sizeof(double)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.rope_sin, rs.size() * sizeof(double)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.rope_cs, rcs.size() * sizeof(double)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.g2s, g2s.size() * sizeof(uint4)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.g3s, g3s.size() * sizeof(uint2)), err, err_len, "tables") &&
         hip_ok(hipMalloc(&c->T.sel8, sel8.size() * sizeof(uint2)), err, err_len, "tables");
    ok = ok && hip_ok(hipMemcpy(c->T.g2, g2.data(), g2.size() * sizeof(uint4), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.g3, g3.data(), g3.size() * sizeof(uint2), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.sel, sel.data(), sel.size() * sizeof(uint2), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.rope_cos, rc.data(), rc.size() * sizeof(double), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.rope_sin, rs.data(), rs.size() * sizeof(double), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.rope_cs, rcs.data(), rcs.size() * sizeof(double), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.g2s, g2s.data(), g2s.size() * sizeof(uint4), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.g3s, g3s.data(), g3s.size() * sizeof(uint2), hipMemcpyHostToDevice), err, err_len, "tables") &&
         hip_ok(hipMemcpy(c->T.sel8, sel8.data(), sel8.size() * sizeof(uint2), hipMemcpyHostToDevice), err, err_len, "tables");
    ok = ok && hip_ok(hipMalloc(&c->st, sizeof(DevState)), err, err_len, "state") &&
         hip_ok(hipMemset(c->st, 0, sizeof(DevState)), err, err_len, "state");
    // tagged exchange buffers start at epoch 0, which no launch uses
    ok = ok && hip_ok(hipMalloc(&c->xch, QXD_XCH_WORDS * 8ull), err, err_len, "exchange buffers") &&
         hip_ok(hipMemset(c->xch, 0, QXD_XCH_WORDS * 8ull), err, err_len, "exchange buffers") &&
         hip_ok(hipMalloc(&c->xpart, 2ull * QXD_PART_WORDS * 8), err, err_len, "exchange buffers") &&
         hip_ok(hipMemset(c->xpart, 0, 2ull * QXD_PART_WORDS * 8), err, err_len, "exchange buffers") &&
         hip_ok(hipMalloc(&c->abort, 4), err, err_len, "abort flag") &&
         hip_ok(hipMemset(c->abort, 0, 4), err, err_len, "abort flag");
    ok = ok && hip_ok(hipEventCreate(&c->e0), err, err_len, "event") && hip_ok(hipEventCreate(&c->e1), err, err_len, "event");
    if (!ok) { qxg_close(c); return 0; }
    *out = c;
    return 1;
}

void qxg_close(qxg_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->s) (void)hipStreamSynchronize(c->s);
    drop_graph(c);
    for (auto &kv : c->tens) free_tensor(kv.second);
    void *bufs[] = {c->T.g2, c->T.g3, c->T.sel, c->T.rope_cos, c->T.rope_sin, c->T.g2s, c->T.g3s, c->T.sel8, c->kc, c->vc, c->ks, c->vs, c->x,
                    c->qkv, c->ctxv, c->h, c->logits, c->vcur, c->attn, c->moe, c->norm, c->layer_dump, c->rlog,
                    c->cand_v, c->top_v, c->cand_i, c->top_i, c->tokens, c->dig, c->st, c->staging,
                    c->xch, c->xpart, c->abort, c->apart, c->route_ids, c->route_w, c->mfold, c->gu_il, c->dn_il, c->head_il, c->dpack,
                    c->T.rope_cs, c->half_dump, c->wsum_dump};
    for (void *p : bufs) if (p) (void)hipFree(p);
    for (void *p : c->arenas) (void)hipFree(p);
    for (void *p : c->pf.all) (void)hipFree(p);
    for (void *p : c->sg.all) (void)hipFree(p);
    for (hipEvent_t e : c->kt.ev) (void)hipEventDestroy(e);
    if (c->e0) (void)hipEventDestroy(c->e0);
    if (c->e1) (void)hipEventDestroy(c->e1);
    if (c->s) (void)hipStreamDestroy(c->s);
    delete c;
}

int qxg_upload_tensor(qxg_ctx *c, const char *name, uint32_t type, const uint64_t dims[4], const void *host,
                      uint64_t nbytes, char *err, uint64_t err_len) {
    if (!c || !name || !dims || !host || !nbytes) { set_err(err, err_len, "invalid argument"); return 0; }
    uint64_t bv = 0, bb = 0;
    if (!block_geom(type, bv, bb)) { set_err(err, err_len, "unsupported ggml type"); return 0; }
    uint64_t elems = 1;
    for (int i = 0; i < 4; ++i) if (dims[i]) elems *= dims[i];
    if (dims[0] % bv || elems / bv * bb != nbytes) { set_err(err, err_len, "tensor byte size inconsistent with dimensions"); return 0; }
    (void)hipSetDevice(c->device);
    drop_graph(c);
    auto it = c->tens.find(name);
    if (it != c->tens.end()) { free_tensor(it->second); c->dev_bytes -= it->second.bytes; c->tens.erase(it); }
    QTensor t;
    t.type = type;
    for (int i = 0; i < 4; ++i) t.dims[i] = dims[i];
    if (!upload_planes(c, t, host, nbytes, err, err_len)) { free_tensor(t); return 0; }
    c->tens[name] = t;
    c->bound = false;
    return 1;
}

int qxg_bind_model(qxg_ctx *c, uint32_t layers, int need_embedding, int need_head, char *err, uint64_t err_len) {
    if (!c) { set_err(err, err_len, "invalid context"); return 0; }
    (void)hipSetDevice(c->device);
    drop_graph(c);
    c->bound = false;
    c->L.assign(layers, LayerW{});
    c->experts = 0;
    bool base = true;
    char msg[256];
    auto bad = [&](const std::string &nm, const char *why) {
        snprintf(msg, sizeof(msg), "%s: %s", nm.c_str(), why);
        set_err(err, err_len, msg);
        return 0;
    };
    for (uint32_t l = 0; l < layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        // accepted formats: the benchmark mix first, then the real checkpoint's per-layer
        // alternatives (attention Q5_K, gate/up IQ2_S, down IQ4_XS or IQ3_S)
        struct { const char *sfx; uint32_t type, alt1, alt2; uint64_t d0, d1; const QTensor **slot; } q[] = {
            {"attn_q.weight", 23, 13, 13, 2048, 4096, &c->L[l].wq}, {"attn_k.weight", 23, 13, 13, 2048, 512, &c->L[l].wk},
            {"attn_v.weight", 23, 13, 13, 2048, 512, &c->L[l].wv}, {"attn_output.weight", 23, 13, 13, 4096, 2048, &c->L[l].wo},
            {"ffn_gate_exps.weight", 17, 22, 22, 2048, 768, &c->L[l].gate}, {"ffn_up_exps.weight", 17, 22, 22, 2048, 768, &c->L[l].up},
            {"ffn_down_exps.weight", 18, 23, 21, 768, 2048, &c->L[l].down}};
        for (auto &e : q) {
            const QTensor *t = find(c, p + e.sfx);
            if (!t) return bad(p + e.sfx, "not uploaded");
            if (t->type != e.type && t->type != e.alt1 && t->type != e.alt2) return bad(p + e.sfx, "unsupported quantization type");
            if (t->dims[0] != e.d0 || t->dims[1] != e.d1) return bad(p + e.sfx, "unexpected shape");
            if (t->type != e.type) base = false;
            *e.slot = t;
        }
        if (c->L[l].gate->type != c->L[l].up->type) return bad(p + "ffn_up_exps.weight", "gate and up experts must share a type");
        const uint32_t E = (uint32_t)c->L[l].gate->dims[2];
        if (E < 8 || E > 128 || c->L[l].up->dims[2] != E || c->L[l].down->dims[2] != E) return bad(p + "ffn_*_exps.weight", "expert count");
        if (l == 0) c->experts = E;
        else if (E != c->experts) return bad(p + "ffn_gate_exps.weight", "expert count differs between layers");
        struct { const char *sfx; uint64_t d0, d1; const float **slot; } f[] = {
            {"attn_norm.weight", 2048, 0, &c->L[l].attn_norm}, {"attn_q_norm.weight", 128, 0, &c->L[l].q_norm},
            {"attn_k_norm.weight", 128, 0, &c->L[l].k_norm}, {"ffn_norm.weight", 2048, 0, &c->L[l].ffn_norm},
            {"ffn_gate_inp.weight", 2048, E, &c->L[l].router}};
        for (auto &e : f) {
            const QTensor *t = find(c, p + e.sfx);
            if (!t) return bad(p + e.sfx, "not uploaded");
            if (t->type != 0 || t->dims[0] != e.d0 || t->dims[1] != e.d1) return bad(p + e.sfx, "must be F32 of the expected shape");
            *e.slot = (const float *)t->p0;
        }
    }
    c->layers = layers;
    c->base_mix = base;
    c->emb = nullptr; c->head = nullptr; c->out_norm = nullptr; c->vocab = 0;
    if (need_embedding) {
        const QTensor *t = find(c, "token_embd.weight");
        if (!t) return bad("token_embd.weight", "not uploaded");
        if (t->type != 12 || t->dims[0] != 2048) return bad("token_embd.weight", "must be Q4_K [2048, vocab]");
        c->emb = t->p0;
        c->vocab = (uint32_t)t->dims[1];
        c->emb_row = t->bytes / t->dims[1];
    }
    if (need_head) {
        const QTensor *t = find(c, "output.weight"), *nw = find(c, "output_norm.weight");
        if (!t || !nw) return bad("output.weight", "output.weight and output_norm.weight must be uploaded");
        if (t->type != 14 || t->dims[0] != 2048) return bad("output.weight", "final head requires Q6_K output.weight");
        if (nw->type != 0 || nw->dims[0] != 2048) return bad("output_norm.weight", "must be F32 [2048]");
        if (c->vocab && c->vocab != t->dims[1]) return bad("output.weight", "vocab differs from token_embd.weight");
        c->head = t;
        c->out_norm = (const float *)nw->p0;
        c->vocab = (uint32_t)t->dims[1];
    }
    // work buffers (re)sized for this binding
    void **bufs[] = {(void **)&c->x, (void **)&c->qkv, (void **)&c->ctxv, (void **)&c->h, (void **)&c->logits,
                     (void **)&c->vcur, (void **)&c->attn, (void **)&c->moe, (void **)&c->norm,
                     (void **)&c->layer_dump, (void **)&c->rlog, (void **)&c->cand_v, (void **)&c->top_v,
                     (void **)&c->cand_i, (void **)&c->top_i, (void **)&c->tokens, (void **)&c->dig, (void **)&c->apart,
                     (void **)&c->route_ids, (void **)&c->route_w, (void **)&c->half_dump, (void **)&c->wsum_dump};
    for (void **b : bufs) if (*b) { (void)hipFree(*b); *b = nullptr; }
    const uint64_t V = c->vocab ? c->vocab : 1;
    const uint64_t sizes[] = {2048 * 4, 5120 * 4, 4096 * 4, 8 * 768 * 4, V * 4, 512 * 4, 2048 * 4, 2048 * 4, 2048 * 4,
                              (uint64_t)(layers ? layers : 1) * 2048 * 4, 128 * 8, TOPK_BLOCKS * QXG_MAX_TOPN * 4,
                              QXG_MAX_TOPN * 4, TOPK_BLOCKS * QXG_MAX_TOPN * 4, QXG_MAX_TOPN * 4,
                              (QXG_MAX_CTX + 2) * 4, (64 * 28 + 4) * 4, QXG_ATT_PART_BYTES,
                              (uint64_t)(layers ? layers : 1) * 8 * 4, (uint64_t)(layers ? layers : 1) * 8 * 8,
                              (uint64_t)(layers ? layers : 1) * 4096 * 4, (uint64_t)(layers ? layers : 1) * 32 * 8};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i)
        if (!hip_ok(hipMalloc(bufs[i], sizes[i]), err, err_len, "work buffers")) return 0;
    if (!hip_ok(hipMemset(c->tokens, 0, sizes[15]), err, err_len, "work buffers")) return 0;
    if (layers && base && !build_arenas(c, err, err_len)) return 0;
    if (c->mfold) { (void)hipFree(c->mfold); c->mfold = nullptr; }
    if (layers && base && !build_router_fold(c, err, err_len)) return 0;
    if (layers && base && !build_expert_interleave(c, err, err_len)) return 0;
    if (layers && base && !build_decode_pack(c, err, err_len)) return 0;
    c->bound = true;
    // one launch of each persistent kernel (both activation modes: the mode may change after
    // binding) with no steps (prologue only): the runtime loads a kernel's code and sets up its
    // first cooperative launch at that launch (≈12 ms measured), which would otherwise fall in
    // the first timed call
    if (persistent(c)) {
        DecodeDumps none;
        const bool q8 = c->q8;
        bool ok = true;
        for (bool mode : {false, true}) {
            c->q8 = mode;
            for (bool chunked : {false, true})
                ok = ok && launch_decode_part(c, chunked, 0, 0, 1, 0, false, none, err, err_len);
        }
        c->q8 = q8;
        if (!ok || !finish(c, err, err_len)) return 0;
    }
    return 1;
}

int qxg_kv_create(qxg_ctx *c, uint32_t layers, uint32_t ctx_tokens, uint32_t kv_format, char *err, uint64_t err_len) {
    if (!c) { set_err(err, err_len, "invalid context"); return 0; }
    if (kv_format != 1) { set_err(err, err_len, "only INT8 KV (kv_format 1) is supported"); return 0; }
    if (!ctx_tokens || ctx_tokens > QXG_MAX_CTX) { set_err(err, err_len, "state loop context must be between 1 and 4096"); return 0; }
    if (!layers) { set_err(err, err_len, "invalid layer count"); return 0; }
    (void)hipSetDevice(c->device);
    drop_graph(c);
    void *b[] = {c->kc, c->vc, c->ks, c->vs};
    for (void *p : b) if (p) (void)hipFree(p);
    c->kc = c->vc = nullptr; c->ks = c->vs = nullptr;
    const uint64_t slots = (uint64_t)layers * ctx_tokens;
    if (!hip_ok(hipMalloc(&c->kc, slots * 512), err, err_len, "kv") || !hip_ok(hipMalloc(&c->vc, slots * 512), err, err_len, "kv") ||
        !hip_ok(hipMalloc(&c->ks, slots * 4), err, err_len, "kv") || !hip_ok(hipMalloc(&c->vs, slots * 4), err, err_len, "kv"))
        return 0;
    // calloc semantics, as the reference (src/qx_format.c:6151-6156)
    if (!hip_ok(hipMemset(c->kc, 0, slots * 512), err, err_len, "kv") || !hip_ok(hipMemset(c->vc, 0, slots * 512), err, err_len, "kv") ||
        !hip_ok(hipMemset(c->ks, 0, slots * 4), err, err_len, "kv") || !hip_ok(hipMemset(c->vs, 0, slots * 4), err, err_len, "kv"))
        return 0;
    c->kv_layers = layers;
    c->att_splits = (ctx_tokens + QXG_ATT_SPLIT - 1) / QXG_ATT_SPLIT;   // every position of the cache
    c->kv_ctx = ctx_tokens;
    return 1;
}

static int kv_copy(qxg_ctx *c, uint32_t layer, uint32_t pos0, uint32_t count, int8_t *k, int8_t *v, float *ksc,
                   float *vsc, bool to_dev, char *err, uint64_t err_len) {
    if (!c || !c->kc) { set_err(err, err_len, "KV cache not created"); return 0; }
    if (layer >= c->kv_layers || pos0 > c->kv_ctx || count > c->kv_ctx - pos0) { set_err(err, err_len, "KV range outside cache"); return 0; }
    (void)hipSetDevice(c->device);
    const uint64_t slot = (uint64_t)layer * c->kv_ctx + pos0;
    const hipMemcpyKind kind = to_dev ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    struct { void *dev; void *host; uint64_t bytes; } m[] = {
        {c->kc + slot * 512, k, (uint64_t)count * 512}, {c->vc + slot * 512, v, (uint64_t)count * 512},
        {c->ks + slot, ksc, (uint64_t)count * 4}, {c->vs + slot, vsc, (uint64_t)count * 4}};
    for (auto &e : m) {
        if (!e.host || !e.bytes) continue;
        hipError_t r = to_dev ? hipMemcpyAsync(e.dev, e.host, e.bytes, kind, c->s) : hipMemcpyAsync(e.host, e.dev, e.bytes, kind, c->s);
        if (!hip_ok(r, err, err_len, "kv copy")) return 0;
    }
    return hip_ok(hipStreamSynchronize(c->s), err, err_len, "kv copy");
}

int qxg_kv_write(qxg_ctx *c, uint32_t layer, uint32_t pos0, uint32_t count, const int8_t *k, const int8_t *v,
                 const float *ks, const float *vs, char *err, uint64_t err_len) {
    return kv_copy(c, layer, pos0, count, (int8_t *)k, (int8_t *)v, (float *)ks, (float *)vs, true, err, err_len);
}

int qxg_kv_read(qxg_ctx *c, uint32_t layer, uint32_t pos0, uint32_t count, int8_t *k, int8_t *v, float *ks,
                float *vs, char *err, uint64_t err_len) {
    return kv_copy(c, layer, pos0, count, k, v, ks, vs, false, err, err_len);
}

int qxg_decode_token(qxg_ctx *c, uint32_t token, uint32_t position, int run_head, float *residual_out,
                     float *layer_out, float *logits, uint32_t top_n, uint32_t *top_ids, double *top_logits,
                     char *err, uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!c->emb) { set_err(err, err_len, "token_embd.weight not bound"); return 0; }
    if (run_head && !c->head) { set_err(err, err_len, "head not bound"); return 0; }
    if (token >= c->vocab) { set_err(err, err_len, "token id out of range"); return 0; }
    if (position >= c->kv_ctx || c->layers > c->kv_layers) { set_err(err, err_len, "position or layers outside KV cache"); return 0; }
    if (top_n == 0) top_n = 1;
    if (top_n > QXG_MAX_TOPN) top_n = QXG_MAX_TOPN;
    (void)hipSetDevice(c->device);
    (void)hipMemcpyAsync(c->tokens, &token, 4, hipMemcpyHostToDevice, c->s);
    write_state(c, position, 0, run_head ? 1 : 2, 0);
    if (persistent(c) && c->layers) {
        // one step of the persistent decode (its head writes every logit), then the top-N
        // of those logits by the per-phase selection kernels
        DecodeDumps d;
        d.layer = c->layer_dump; d.res = c->x; d.rids = c->route_ids; d.rw = c->route_w; d.half = c->half_dump;
        d.wsum = c->wsum_dump;
        d.norm = run_head ? c->norm : nullptr;
        d.logits = run_head ? c->logits : nullptr;
        if (!launch_decode(c, 1, run_head ? 1 : 2, position, false, d, err, err_len)) return 0;
        if (run_head) {
            hipLaunchKernelGGL(qxk_topk, dim3(TOPK_BLOCKS), dim3(256), 0, c->s, c->logits, c->vocab, top_n, c->cand_v,
                               c->cand_i, c->top_v, c->top_i, c->tokens, c->st);
            hipLaunchKernelGGL(qxk_topk_merge, dim3(1), dim3(256), 0, c->s, (const float *)c->cand_v,
                               (const uint32_t *)c->cand_i, (uint32_t)TOPK_BLOCKS, top_n, c->top_v, c->top_i, c->tokens, c->st);
        }
    } else {
        hipLaunchKernelGGL(qxk_embed, dim3(1), dim3(256), 0, c->s, c->emb, c->emb_row, c->tokens, c->st, c->x);
        for (uint32_t l = 0; l < c->layers; ++l) {
            launch_attention(c, l, c->x, c->half_dump + 4096ull * l, nullptr, c->wsum_dump + 32ull * l);
            launch_moe(c, l, c->x, c->half_dump + 4096ull * l + 2048);
            if (layer_out)
                (void)hipMemcpyAsync(c->layer_dump + 2048ull * l, c->x, 2048 * 4, hipMemcpyDeviceToDevice, c->s);
        }
        if (run_head) launch_head(c, top_n, c->norm);
    }
    if (!finish(c, err, err_len)) return 0;
    if (residual_out && !hip_ok(hipMemcpy(residual_out, c->x, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (layer_out && !hip_ok(hipMemcpy(layer_out, c->layer_dump, 2048ull * 4 * c->layers, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (!run_head) return 1;
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (logits && !hip_ok(hipMemcpy(logits, c->logits, (uint64_t)c->vocab * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    float tv[QXG_MAX_TOPN];
    uint32_t ti[QXG_MAX_TOPN];
    if (!hip_ok(hipMemcpy(tv, c->top_v, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read") ||
        !hip_ok(hipMemcpy(ti, c->top_i, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    for (uint32_t i = 0; i < top_n; ++i) {
        if (top_ids) top_ids[i] = ti[i];
        if (top_logits) top_logits[i] = (double)tv[i];
    }
    if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
    return 1;
}

int qxg_generate(qxg_ctx *c, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_gen, uint32_t pos0,
                 uint32_t *tokens_out, float *elapsed_ms, char *err, uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!c->emb || !c->head) { set_err(err, err_len, "generation needs token_embd.weight and output.weight bound"); return 0; }
    if (!prompt || !n_prompt || !n_gen) { set_err(err, err_len, "generation needs >= 1 prompt token and >= 1 generated token"); return 0; }
    const uint64_t steps = (uint64_t)n_prompt + n_gen - 1;
    if (pos0 + steps > c->kv_ctx || c->layers > c->kv_layers) { set_err(err, err_len, "prompt plus generation exceeds the KV context"); return 0; }
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= c->vocab) { set_err(err, err_len, "prompt token out of range"); return 0; }
    (void)hipSetDevice(c->device);
    (void)hipMemcpyAsync(c->tokens, prompt, (uint64_t)n_prompt * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, pos0, 0, n_prompt, 0);
    c->kt.used = 0;
    if (persistent(c) && c->layers) {   // every step in one cooperative launch
        (void)hipEventRecord(c->e0, c->s);
        if (!launch_decode(c, (uint32_t)steps, n_prompt, pos0, false, DecodeDumps(), err, err_len)) return 0;
        (void)hipEventRecord(c->e1, c->s);
        if (!finish(c, err, err_len)) return 0;
        if (elapsed_ms) (void)hipEventElapsedTime(elapsed_ms, c->e0, c->e1);
        DevState h;
        if (!read_state(c, h, err, err_len)) return 0;
        if (tokens_out && !hip_ok(hipMemcpy(tokens_out, c->tokens + n_prompt, (uint64_t)n_gen * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
        if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
        return 1;
    }
    // in-situ kernel timing records events per launch, and QXG_EAGER asks for plain launches
    // (kernel tracers): run eagerly
    const bool use_graph = c->kt.which < 0 && !c->eager;
    // attention splits for the positions this call reaches (the graph is recorded again
    // when that count changes); restored to the whole cache's afterwards
    const uint32_t all_splits = c->att_splits;
    c->att_splits = (uint32_t)((pos0 + steps + QXG_ATT_SPLIT - 1) / QXG_ATT_SPLIT);
    struct Restore {
        qxg_ctx *c;
        uint32_t v;
        ~Restore() { c->att_splits = v; }
    } restore{c, all_splits};
    if (use_graph && c->graph_exec && c->graph_splits != c->att_splits) drop_graph(c);
    if (use_graph && !c->graph_exec) {
        c->graph_splits = c->att_splits;
        // every kernel reads the position/step from the device state, so one recorded
        // step serves all steps; no memset nodes are recorded
        if (!hip_ok(hipStreamBeginCapture(c->s, hipStreamCaptureModeThreadLocal), err, err_len, "capture")) return 0;
        launch_step(c, 1, false);
        hipLaunchKernelGGL(qxk_advance, dim3(1), dim3(64), 0, c->s, c->st, (const double *)c->T.rope_cos,
                           (const double *)c->T.rope_sin);
        hipGraph_t g = nullptr;
        if (!hip_ok(hipStreamEndCapture(c->s, &g), err, err_len, "capture")) return 0;
        c->graph = g;
        if (!hip_ok(hipGraphInstantiate(&c->graph_exec, g, nullptr, nullptr, 0), err, err_len, "graph instantiate")) {
            drop_graph(c);
            return 0;
        }
    }
    (void)hipEventRecord(c->e0, c->s);
    for (uint64_t s = 0; s < steps; ++s) {
        if (use_graph) {
            if (!hip_ok(hipGraphLaunch(c->graph_exec, c->s), err, err_len, "graph launch")) return 0;
        } else {
            launch_step(c, 1, false);
            hipLaunchKernelGGL(qxk_advance, dim3(1), dim3(64), 0, c->s, c->st, (const double *)c->T.rope_cos,
                           (const double *)c->T.rope_sin);
        }
    }
    (void)hipEventRecord(c->e1, c->s);
    if (!finish(c, err, err_len)) return 0;
    if (elapsed_ms) (void)hipEventElapsedTime(elapsed_ms, c->e0, c->e1);
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (tokens_out && !hip_ok(hipMemcpy(tokens_out, c->tokens + n_prompt, (uint64_t)n_gen * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
    return 1;
}

int qxg_dequant_blocks(qxg_ctx *c, uint32_t type, const void *raw, uint64_t nblocks, float *out, char *err, uint64_t err_len) {
    if (!c || !raw || !out || !nblocks) { set_err(err, err_len, "invalid argument"); return 0; }
    uint64_t bv = 0, bb = 0;
    if (!block_geom(type, bv, bb) || type == 0) { set_err(err, err_len, "unsupported GGML type for decode-block"); return 0; }
    (void)hipSetDevice(c->device);
    QTensor t;
    t.type = type;
    t.dims[0] = 256 * nblocks;
    const uint64_t before = c->dev_bytes;
    if (!upload_planes(c, t, raw, nblocks * bb, err, err_len)) { free_tensor(t); c->dev_bytes = before; return 0; }
    c->dev_bytes = before;
    float *d = nullptr;
    int ok = hip_ok(hipMalloc(&d, nblocks * 256 * 4), err, err_len, "hipMalloc");
    if (ok) {
        hipLaunchKernelGGL(qxk_dequant, dim3((unsigned)nblocks), dim3(256), 0, c->s, type, t.p0, t.p1, t.p2, t.d, c->T,
                           nblocks, d);
        ok = finish(c, err, err_len) && hip_ok(hipMemcpy(out, d, nblocks * 256 * 4, hipMemcpyDeviceToHost), err, err_len, "read");
    }
    if (d) (void)hipFree(d);
    free_tensor(t);
    return ok;
}

int qxg_int8_quantize(qxg_ctx *c, const float *x, uint32_t n, int8_t *codes, float *scale, char *err, uint64_t err_len) {
    if (!c || !x || !codes || !scale || !n || n > 4096) { set_err(err, err_len, "invalid argument"); return 0; }
    (void)hipSetDevice(c->device);
    float *dx = nullptr;
    int ok = hip_ok(hipMalloc(&dx, n * 4 + 4 + n), err, err_len, "hipMalloc");
    if (ok) {
        float *dsc = dx + n;
        int8_t *dc = (int8_t *)(dx + n + 1);
        ok = hip_ok(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->s), err, err_len, "copy");
        if (ok) {
            hipLaunchKernelGGL(qxk_int8_row, dim3(1), dim3(256), 0, c->s, dx, n, dc, dsc);
            ok = finish(c, err, err_len) && hip_ok(hipMemcpy(codes, dc, n, hipMemcpyDeviceToHost), err, err_len, "read") &&
                 hip_ok(hipMemcpy(scale, dsc, 4, hipMemcpyDeviceToHost), err, err_len, "read");
        }
    }
    if (dx) (void)hipFree(dx);
    return ok;
}

int qxg_dequant_blocks_static(qxg_ctx *c, uint32_t type, const void *raw_dev, uint64_t nblocks, float *out_dev, char *err,
                              uint64_t err_len) {
    if (!c || !raw_dev || !out_dev || !nblocks) { set_err(err, err_len, "invalid argument"); return 0; }
    uint64_t bv = 0, bb = 0;
    if (!block_geom(type, bv, bb) || type == 0) { set_err(err, err_len, "unsupported GGML type for decode-block"); return 0; }
    if (nblocks > QXG_STATIC_MAX_BLOCKS) {
        if (err && err_len)
            snprintf(err, (size_t)err_len, "qxg_dequant_blocks_static: %llu blocks; the static workspace holds at most %u",
                     (unsigned long long)nblocks, QXG_STATIC_MAX_BLOCKS);
        return 0;
    }
    if (!c->scratch) { set_err(err, err_len, "static workspace address not set"); return 0; }
    // calls on one GPU share its workspace: held from the repack until the call has finished,
    // so overlapping calls (other contexts, other threads) run one after another
    std::lock_guard<std::mutex> use(scratch_use(c->device));
    (void)hipSetDevice(c->device);
    const uint8_t *raw = (const uint8_t *)raw_dev;
    uint8_t *p0 = c->scratch + SCR_P0, *p1 = c->scratch + SCR_P1, *p2 = c->scratch + SCR_P2;
    uint16_t *d = (uint16_t *)(c->scratch + SCR_D);
    if (type == 12) {   // Q4_K is read in its original layout: straight from the caller's blocks
        hipLaunchKernelGGL(qxk_dequant, dim3((unsigned)nblocks), dim3(256), 0, c->s, type, raw, (const uint8_t *)nullptr,
                           (const uint8_t *)nullptr, (const uint16_t *)nullptr, c->T, nblocks, out_dev);
    } else {
        hipLaunchKernelGGL(qxk_repack, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, c->s, type, raw, nblocks, p0,
                           p1, p2, d);
        hipLaunchKernelGGL(qxk_dequant, dim3((unsigned)nblocks), dim3(256), 0, c->s, type, (const uint8_t *)p0,
                           (const uint8_t *)p1, (const uint8_t *)p2, (const uint16_t *)d, c->T, nblocks, out_dev);
    }
    return finish(c, err, err_len);
}

int qxg_q8k_quantize(qxg_ctx *c, const float *x, uint32_t n, void *blocks_out, char *err, uint64_t err_len) {
    if (!c || !x || !blocks_out) { set_err(err, err_len, "invalid argument"); return 0; }
    if (!n || n % 256u) { set_err(err, err_len, "Q8_K activation length must be a non-zero multiple of 256"); return 0; }
    if (n > 4096u) { set_err(err, err_len, "Q8_K activation workspace is too small"); return 0; }
    (void)hipSetDevice(c->device);
    const uint64_t out_bytes = (uint64_t)n / 256 * 292;
    uint8_t *buf = nullptr;
    if (!hip_ok(hipMalloc(&buf, n * 4ull + out_bytes + 4), err, err_len, "hipMalloc")) return 0;
    float *dx = (float *)buf;
    uint8_t *dout = buf + n * 4ull;
    uint32_t *dbad = (uint32_t *)(dout + out_bytes);
    uint32_t bad = 0;
    int ok = hip_ok(hipMemcpy(dx, x, n * 4ull, hipMemcpyHostToDevice), err, err_len, "upload") &&
             hip_ok(hipMemset(dbad, 0, 4), err, err_len, "memset");
    if (ok) {
        hipLaunchKernelGGL(qxk_q8k, dim3((n / 8 + 255) / 256), dim3(256), 0, c->s, (const float *)dx, n, dout, dbad);
        ok = finish(c, err, err_len) && hip_ok(hipMemcpy(blocks_out, dout, out_bytes, hipMemcpyDeviceToHost), err, err_len, "read") &&
             hip_ok(hipMemcpy(&bad, dbad, 4, hipMemcpyDeviceToHost), err, err_len, "read");
    }
    (void)hipFree(buf);
    if (ok && bad) { set_err(err, err_len, "Q8_K activation contains NaN or Inf"); return 0; }
    return ok;
}

int qxg_embed_token(qxg_ctx *c, uint32_t token, float *x_out, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!c->emb) { set_err(err, err_len, "token_embd.weight not bound"); return 0; }
    if (token >= c->vocab || !x_out) { set_err(err, err_len, "token id out of range"); return 0; }
    (void)hipSetDevice(c->device);
    (void)hipMemcpyAsync(c->tokens, &token, 4, hipMemcpyHostToDevice, c->s);
    write_state(c, 0, 0, 1, 1);
    hipLaunchKernelGGL(qxk_embed, dim3(1), dim3(256), 0, c->s, c->emb, c->emb_row, c->tokens, c->st, c->x);
    if (!finish(c, err, err_len)) return 0;
    return hip_ok(hipMemcpy(x_out, c->x, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read");
}

namespace {
bool stage_buffers(qxg_ctx *c, char *err, uint64_t n) {
    auto &g = c->sg;
    if (g.bad) return true;
    auto get = [&](void **p, uint64_t bytes) {
        if (!hip_ok(hipMalloc(p, bytes), err, n, "stage buffer")) return false;
        g.all.push_back(*p);
        return true;
    };
    return get((void **)&g.wsum, 32 * 8) && get((void **)&g.norm, 2048 * 4) && get((void **)&g.route, (2 * 128 + 25) * 4) &&
           get((void **)&g.gu, 2 * QXG_TOPK * QXG_FFN * 4) && get((void **)&g.down, QXG_TOPK * 2048 * 4) &&
           get((void **)&g.wdown, QXG_TOPK * 2048 * 4) && get((void **)&g.bad, 4);
}
}  // namespace

int qxg_attention_layer(qxg_ctx *c, uint32_t layer, uint32_t position, const float *x_in, float *attn_out,
                        float *kqv_out, float *vcur_out, char *err, uint64_t err_len) {
    return qxg_attention_layer_ex(c, layer, position, x_in, attn_out, kqv_out, vcur_out, nullptr, err, err_len);
}

int qxg_attention_layer_ex(qxg_ctx *c, uint32_t layer, uint32_t position, const float *x_in, float *attn_out,
                           float *kqv_out, float *vcur_out, double *head_weight_sums, char *err, uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!x_in || layer >= c->layers || layer >= c->kv_layers || position >= c->kv_ctx) { set_err(err, err_len, "invalid attention layer argument"); return 0; }
    (void)hipSetDevice(c->device);
    if (head_weight_sums && !stage_buffers(c, err, err_len)) return 0;
    (void)hipMemcpyAsync(c->x, x_in, 2048 * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, position, 0, 1, 1);
    launch_attention(c, layer, c->x, c->attn, c->vcur, head_weight_sums ? c->sg.wsum : nullptr);
    if (!finish(c, err, err_len)) return 0;
    if (head_weight_sums && !hip_ok(hipMemcpy(head_weight_sums, c->sg.wsum, 32 * 8, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (attn_out && !hip_ok(hipMemcpy(attn_out, c->attn, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (kqv_out && !hip_ok(hipMemcpy(kqv_out, c->ctxv, 4096 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (vcur_out && !hip_ok(hipMemcpy(vcur_out, c->vcur, 512 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    return 1;
}

int qxg_moe_layer(qxg_ctx *c, uint32_t layer, const float *ffn_inp, float *layer_out, float *moe_out, uint32_t ids[8],
                  double weights[8], char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!ffn_inp || layer >= c->layers) { set_err(err, err_len, "invalid MoE layer argument"); return 0; }
    (void)hipSetDevice(c->device);
    (void)hipMemcpyAsync(c->x, ffn_inp, 2048 * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, 0, 0, 1, 1);
    launch_moe(c, layer, c->x, c->moe);
    if (!finish(c, err, err_len)) return 0;
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (layer_out && !hip_ok(hipMemcpy(layer_out, c->x, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (moe_out && !hip_ok(hipMemcpy(moe_out, c->moe, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    for (int r = 0; r < 8; ++r) {
        if (ids) ids[r] = h.moe_ids[r];
        if (weights) weights[r] = h.moe_w[r];
    }
    return 1;
}

int qxg_attention_stage(qxg_ctx *c, uint32_t layer, int f16_kv, const float *x_in, float *norm_out, float *vcur_out,
                        float *kqv_out, float *attn_out, float *ffn_inp_out, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!x_in || layer >= c->layers) { set_err(err, err_len, "invalid attention stage layer or dimensions"); return 0; }
    (void)hipSetDevice(c->device);
    if (!stage_buffers(c, err, err_len)) return 0;
    const LayerW &w = c->L[layer];
    (void)hipMemcpyAsync(c->x, x_in, 2048 * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, 0, 0, 1, 1);
    hipLaunchKernelGGL(qxp_norm, dim3(1), dim3(256), 0, c->s, (const float *)c->x, w.attn_norm, 1u, c->sg.norm);
    qxl_qkv(c->s, c->x, w.attn_norm, w.wq, w.wk, w.wv, c->qkv, c->st, c->q8);
    hipLaunchKernelGGL(qxk_stage_ctx, dim3(1), dim3(256), 0, c->s, (const float *)c->qkv, (uint32_t)(f16_kv != 0), c->ctxv);
    qxl_oproj(c->s, c->ctxv, w.wo, c->x, c->attn, c->st, c->q8);   // x becomes ffn_inp, attn the O output
    if (!finish(c, err, err_len)) return 0;
    std::vector<float> fi(2048), ao(2048);
    if (!hip_ok(hipMemcpy(fi.data(), c->x, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read") ||
        !hip_ok(hipMemcpy(ao.data(), c->attn, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    for (int i = 0; i < 2048; ++i)
        if (!std::isfinite(ao[i]) || !std::isfinite(fi[i])) { set_err(err, err_len, "non-finite attention stage output"); return 0; }
    if (norm_out && !hip_ok(hipMemcpy(norm_out, c->sg.norm, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (vcur_out && !hip_ok(hipMemcpy(vcur_out, c->qkv + 4608, 512 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (kqv_out && !hip_ok(hipMemcpy(kqv_out, c->ctxv, 4096 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (attn_out) memcpy(attn_out, ao.data(), 2048 * 4);
    if (ffn_inp_out) memcpy(ffn_inp_out, fi.data(), 2048 * 4);
    return 1;
}

int qxg_moe_stage(qxg_ctx *c, uint32_t layer, const float *x_in, float *out, uint32_t ids[8], char *err,
                  uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!x_in || !out || layer >= c->layers) { set_err(err, err_len, "invalid MoE stage layer"); return 0; }
    if (c->experts < 8 || c->experts > 128) { set_err(err, err_len, "unsupported MoE stage tensor layout"); return 0; }
    (void)hipSetDevice(c->device);
    if (!stage_buffers(c, err, err_len)) return 0;
    const LayerW &w = c->L[layer];
    const uint32_t E = c->experts;
    (void)hipMemcpyAsync(c->x, x_in, 2048 * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, 0, 0, 1, 1);
    hipLaunchKernelGGL(qxp_norm, dim3(1), dim3(256), 0, c->s, (const float *)c->x, w.ffn_norm, 1u, c->sg.norm);
    hipLaunchKernelGGL(qxk_router, dim3(E), dim3(256), 0, c->s, (const float *)c->x, w.ffn_norm, w.router, E, c->rlog);
    hipLaunchKernelGGL(qxk_stage_route, dim3(1), dim3(64), 0, c->s, (const double *)c->rlog, E, c->sg.route, c->st, c->sg.bad);
    qxl_gate_up(c->s, c->x, w.ffn_norm, w.gate, w.up, c->T, c->rlog, E, c->st, c->h, c->route_ids + 8 * layer,
                c->route_w + 8 * layer, c->q8, Timer(), c->st->moe_ids, c->sg.gu);
    qxl_down(c->s, c->h, w.down, c->T, c->st, c->x, c->moe, c->q8, Timer(), c->sg.down, c->sg.wdown);
    if (!finish(c, err, err_len)) return 0;
    uint32_t bad = 0;
    if (!hip_ok(hipMemcpy(&bad, c->sg.bad, 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (bad) {
        set_err(err, err_len, bad == 1 ? "non-finite MoE router logit" : bad == 2 ? "invalid MoE router softmax"
                                                                       : "invalid selected MoE weights");
        return 0;
    }
    const uint64_t F8 = QXG_TOPK * QXG_FFN;
    float *o = out;
    auto rd = [&](float *dst, const void *src, uint64_t nf) {
        return hip_ok(hipMemcpy(dst, src, nf * 4, hipMemcpyDeviceToHost), err, err_len, "read");
    };
    if (!rd(o, c->sg.norm, 2048)) return 0;
    o += 2048;
    if (!rd(o, c->sg.route, 2 * E + 25)) return 0;
    o += 2 * E + 25;
    if (!rd(o, c->sg.gu, 2 * F8) || !rd(o + 2 * F8, c->h, F8)) return 0;
    o += 3 * F8;
    if (!rd(o, c->sg.down, QXG_TOPK * 2048) || !rd(o + QXG_TOPK * 2048, c->sg.wdown, QXG_TOPK * 2048)) return 0;
    if (ids) {
        DevState h;
        if (!read_state(c, h, err, err_len)) return 0;
        for (int r = 0; r < 8; ++r) ids[r] = h.moe_ids[r];
    }
    return 1;
}

int qxg_final_head(qxg_ctx *c, const float *residual, float *norm_out, float *logits, uint32_t top_n,
                   uint32_t *top_ids, double *top_logits, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!c->head) { set_err(err, err_len, "final head requires Q6_K output.weight"); return 0; }
    if (!residual) { set_err(err, err_len, "invalid final head argument"); return 0; }
    if (top_n == 0) top_n = 1;
    if (top_n > QXG_MAX_TOPN) top_n = QXG_MAX_TOPN;
    (void)hipSetDevice(c->device);
    (void)hipMemcpyAsync(c->x, residual, 2048 * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, 0, 0, 1, 1);
    launch_head(c, top_n, c->norm);
    if (!finish(c, err, err_len)) return 0;
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (norm_out && !hip_ok(hipMemcpy(norm_out, c->norm, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (logits && !hip_ok(hipMemcpy(logits, c->logits, (uint64_t)c->vocab * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    float tv[QXG_MAX_TOPN];
    uint32_t ti[QXG_MAX_TOPN];
    if (!hip_ok(hipMemcpy(tv, c->top_v, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read") ||
        !hip_ok(hipMemcpy(ti, c->top_i, top_n * 4, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    for (uint32_t i = 0; i < top_n; ++i) {
        if (top_ids) top_ids[i] = ti[i];
        if (top_logits) top_logits[i] = (double)tv[i];
    }
    if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
    return 1;
}

int qxg_time_kernel(qxg_ctx *c, int which, uint32_t layer, uint32_t iters, float *avg_ms, char *err, uint64_t err_len) {
    if (!check_ready(c, which == 5 || which == 2, err, err_len)) return 0;
    if (which < 0 || which > 6 || !iters || layer >= c->layers) { set_err(err, err_len, "invalid timing argument"); return 0; }
    if (which == 4 && !c->head) { set_err(err, err_len, "head not bound"); return 0; }
    (void)hipSetDevice(c->device);
    // rotate over layers so repeated launches stream distinct weights (> the 256 MB MALL)
    (void)hipEventRecord(c->e0, c->s);
    for (uint32_t i = 0; i < iters; ++i) {
        const uint32_t l = (layer + i) % c->layers;
        const LayerW &w = c->L[l];
        switch (which) {
        case 0:
            qxl_gate_up(c->s, c->x, w.ffn_norm, w.gate, w.up, c->T, c->rlog, c->experts, c->st, c->h, c->route_ids + 8 * l,
                        c->route_w + 8 * l, c->q8);
            break;
        case 1: qxl_down(c->s, c->h, w.down, c->T, c->st, c->attn, nullptr, c->q8); break;
        case 2: qxl_qkv(c->s, c->x, w.attn_norm, w.wq, w.wk, w.wv, c->qkv, c->st, c->q8); break;
        case 3: qxl_oproj(c->s, c->ctxv, w.wo, c->attn, nullptr, c->st, c->q8); break;
        case 4: qxl_head(c->s, c->x, c->out_norm, c->head, c->vocab, c->st, c->logits, nullptr, c->dig, c->q8); break;
        case 5:
            hipLaunchKernelGGL(qxk_attn, dim3(32, c->att_splits), dim3(256), 0, c->s, c->qkv, w.q_norm, w.k_norm, c->T,
                               c->kc, c->vc, c->ks, c->vs, l % c->kv_layers, c->kv_ctx, std::sqrt(128.0), c->st,
                               c->ctxv, c->apart, nullptr, nullptr);
            if (c->att_splits > 1)
                hipLaunchKernelGGL(qxk_attn_merge, dim3(32), dim3(128), 0, c->s, (const DevState *)c->st,
                                   (const float *)c->apart, c->ctxv, nullptr);
            break;
        case 6:
            hipLaunchKernelGGL(qxk_router, dim3(c->experts), dim3(256), 0, c->s, (const float *)c->x, w.ffn_norm,
                               w.router, c->experts, c->rlog);
            break;
        }
    }
    (void)hipEventRecord(c->e1, c->s);
    if (!finish(c, err, err_len)) return 0;
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, c->e0, c->e1);
    if (avg_ms) *avg_ms = ms / (float)iters;
    return 1;
}

uint64_t qxg_device_bytes(const qxg_ctx *c) { return c ? c->dev_bytes : 0; }

int qxg_persistent_path(const qxg_ctx *c) { return c && c->bound && c->layers && persistent(c) ? 1 : 0; }

int qxg_generate_recorded(qxg_ctx *c, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_gen, uint32_t pos0,
                          uint32_t top_n, uint32_t *tokens_out, float *layer_out, float *attn_out, float *moe_out,
                          uint32_t *ids_out, double *weights_out, double *head_sums_out, float *norm_out, float *logits_out,
                          uint32_t *top_ids, double *top_logits, double *step_ms, float *elapsed_ms, char *err,
                          uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!persistent(c) || !c->layers) { set_err(err, err_len, "recorded generation runs the persistent decode only"); return 0; }
    if (!prompt || !n_prompt || !n_gen) { set_err(err, err_len, "generation needs >= 1 prompt token and >= 1 generated token"); return 0; }
    const uint64_t steps = (uint64_t)n_prompt + n_gen - 1, L = c->layers, V = c->vocab;
    if (pos0 + steps > c->kv_ctx || c->layers > c->kv_layers) { set_err(err, err_len, "prompt plus generation exceeds the KV context"); return 0; }
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= c->vocab) { set_err(err, err_len, "prompt token out of range"); return 0; }
    if (top_n == 0) top_n = 1;
    if (top_n > QXG_MAX_TOPN) top_n = QXG_MAX_TOPN;
    (void)hipSetDevice(c->device);
    // one slot per step of every record (device), freed at the end of the call
    const uint64_t n_lay = steps * L * 2048, n_half = steps * L * 4096, n_ids = steps * L * 8, n_ws = steps * L * 32;
    const uint64_t n_res = steps * 2048, n_lg = steps * V, n_top = steps * QXG_MAX_TOPN;
    float *d_lay = nullptr, *d_half = nullptr, *d_res = nullptr, *d_norm = nullptr, *d_lg = nullptr, *d_tv = nullptr;
    uint32_t *d_ids = nullptr, *d_ti = nullptr, *d_tok = nullptr;
    double *d_w = nullptr, *d_ws = nullptr;
    uint64_t *d_time = nullptr;
    DevState *d_post = nullptr;
    struct Frees {
        std::vector<void *> p;
        ~Frees() { for (void *q : p) if (q) (void)hipFree(q); }
    } frees;
    auto get = [&](void **q, uint64_t bytes) {
        if (!hip_ok(hipMalloc(q, bytes), err, err_len, "record buffers")) return false;
        frees.p.push_back(*q);
        return true;
    };
    if (!get((void **)&d_lay, n_lay * 4) || !get((void **)&d_half, n_half * 4) || !get((void **)&d_res, n_res * 4) ||
        !get((void **)&d_norm, n_res * 4) || !get((void **)&d_lg, n_lg * 4) || !get((void **)&d_tv, n_top * 4) ||
        !get((void **)&d_ids, n_ids * 4) || !get((void **)&d_ti, n_top * 4) || !get((void **)&d_tok, 8) ||
        !get((void **)&d_w, n_ids * 8) || !get((void **)&d_ws, n_ws * 8) || !get((void **)&d_post, sizeof(DevState)) ||
        !get((void **)&d_time, (steps + 1) * 8))
        return 0;
    // the prompt steps before the last write no head records: their slots read back as zeros
    if (!hip_ok(hipMemsetAsync(d_norm, 0, n_res * 4, c->s), err, err_len, "record buffers") ||
        !hip_ok(hipMemsetAsync(d_lg, 0, n_lg * 4, c->s), err, err_len, "record buffers") ||
        !hip_ok(hipMemsetAsync(d_tv, 0, n_top * 4, c->s), err, err_len, "record buffers") ||
        !hip_ok(hipMemsetAsync(d_ti, 0, n_top * 4, c->s), err, err_len, "record buffers"))
        return 0;
    (void)hipMemcpyAsync(c->tokens, prompt, (uint64_t)n_prompt * 4, hipMemcpyHostToDevice, c->s);
    write_state(c, pos0, 0, n_prompt, 0);
    DecodeDumps d;
    d.layer = d_lay; d.res = d_res; d.rids = d_ids; d.rw = d_w; d.half = d_half; d.wsum = d_ws; d.norm = d_norm; d.logits = d_lg;
    d.rec_all = true;
    d.time = d_time;
    (void)hipEventRecord(c->e0, c->s);
    if (!launch_decode(c, (uint32_t)steps, n_prompt, pos0, false, d, err, err_len)) return 0;
    (void)hipEventRecord(c->e1, c->s);
    // each head step's top-N from its recorded logits (the per-phase selection kernels, on a
    // scratch state that marks a generate step and a scratch token pair)
    DevState post{};
    post.n_prompt = 1;
    (void)hipMemcpyAsync(d_post, &post, sizeof(post), hipMemcpyHostToDevice, c->s);
    for (uint64_t s = (n_prompt > 0 ? n_prompt - 1 : 0); s < steps; ++s) {
        hipLaunchKernelGGL(qxk_topk, dim3(TOPK_BLOCKS), dim3(256), 0, c->s, (const float *)(d_lg + s * V), c->vocab, top_n,
                           c->cand_v, c->cand_i, d_tv + s * QXG_MAX_TOPN, d_ti + s * QXG_MAX_TOPN, d_tok, d_post);
        hipLaunchKernelGGL(qxk_topk_merge, dim3(1), dim3(256), 0, c->s, (const float *)c->cand_v, (const uint32_t *)c->cand_i,
                           (uint32_t)TOPK_BLOCKS, top_n, d_tv + s * QXG_MAX_TOPN, d_ti + s * QXG_MAX_TOPN, d_tok, d_post);
    }
    if (!finish(c, err, err_len)) return 0;
    if (elapsed_ms) (void)hipEventElapsedTime(elapsed_ms, c->e0, c->e1);
    DevState h;
    if (!read_state(c, h, err, err_len)) return 0;
    if (h.nonfinite) { write_state(c, 0, 0, 0, 0); set_err(err, err_len, "non-finite final logit"); return 0; }
    auto rd = [&](void *dst, const void *src, uint64_t bytes) {
        return !dst || hip_ok(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), err, err_len, "read");
    };
    if (!rd(tokens_out, c->tokens, (steps + 1) * 4) || !rd(layer_out, d_lay, n_lay * 4) || !rd(ids_out, d_ids, n_ids * 4) ||
        !rd(weights_out, d_w, n_ids * 8) || !rd(head_sums_out, d_ws, n_ws * 8) || !rd(norm_out, d_norm, n_res * 4) ||
        !rd(logits_out, d_lg, n_lg * 4))
        return 0;
    if (attn_out && !hip_ok(hipMemcpy2D(attn_out, 2048 * 4, d_half, 4096 * 4, 2048 * 4, steps * L, hipMemcpyDeviceToHost),
                            err, err_len, "read"))
        return 0;
    if (moe_out && !hip_ok(hipMemcpy2D(moe_out, 2048 * 4, d_half + 2048, 4096 * 4, 2048 * 4, steps * L, hipMemcpyDeviceToHost),
                           err, err_len, "read"))
        return 0;
    if (step_ms) {   // the device clock (100 MHz) of each step's start and the end, from the first start
        std::vector<uint64_t> t(steps + 1);
        if (!rd(t.data(), d_time, (steps + 1) * 8)) return 0;
        for (uint64_t s = 0; s <= steps; ++s) step_ms[s] = (double)(int64_t)(t[s] - t[0]) * 1e-5;
    }
    if (top_ids || top_logits) {
        std::vector<float> tv(n_top);
        std::vector<uint32_t> ti(n_top);
        if (!rd(tv.data(), d_tv, n_top * 4) || !rd(ti.data(), d_ti, n_top * 4)) return 0;
        for (uint64_t s = 0; s < steps; ++s)
            for (uint32_t i = 0; i < top_n; ++i) {
                if (top_ids) top_ids[s * top_n + i] = ti[s * QXG_MAX_TOPN + i];
                if (top_logits) top_logits[s * top_n + i] = (double)tv[s * QXG_MAX_TOPN + i];
            }
    }
    return 1;
}

int qxg_decode_routing(qxg_ctx *c, uint32_t layers, uint32_t *ids, double *weights, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!layers || layers > c->layers || !ids || !weights) { set_err(err, err_len, "invalid argument"); return 0; }
    (void)hipSetDevice(c->device);
    return hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream") &&
           hip_ok(hipMemcpy(ids, c->route_ids, (uint64_t)layers * 8 * 4, hipMemcpyDeviceToHost), err, err_len, "read") &&
           hip_ok(hipMemcpy(weights, c->route_w, (uint64_t)layers * 8 * 8, hipMemcpyDeviceToHost), err, err_len, "read");
}

int qxg_decode_halves(qxg_ctx *c, uint32_t layers, float *attn_out, float *moe_out, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!layers || layers > c->layers) { set_err(err, err_len, "invalid argument"); return 0; }
    (void)hipSetDevice(c->device);
    if (!hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream")) return 0;
    // one strided copy per half ([layer][attention | MoE] on the device)
    return (!attn_out || hip_ok(hipMemcpy2D(attn_out, 2048 * 4, c->half_dump, 4096 * 4, 2048 * 4, layers, hipMemcpyDeviceToHost),
                                err, err_len, "read")) &&
           (!moe_out || hip_ok(hipMemcpy2D(moe_out, 2048 * 4, c->half_dump + 2048, 4096 * 4, 2048 * 4, layers,
                                           hipMemcpyDeviceToHost), err, err_len, "read"));
}

int qxg_decode_final_norm(qxg_ctx *c, float *norm_out, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!norm_out) { set_err(err, err_len, "invalid argument"); return 0; }
    (void)hipSetDevice(c->device);
    return hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream") &&
           hip_ok(hipMemcpy(norm_out, c->norm, 2048 * 4, hipMemcpyDeviceToHost), err, err_len, "read");
}

int qxg_decode_head_sums(qxg_ctx *c, uint32_t layers, double *sums, char *err, uint64_t err_len) {
    if (!check_ready(c, false, err, err_len)) return 0;
    if (!layers || layers > c->layers || !sums) { set_err(err, err_len, "invalid argument"); return 0; }
    (void)hipSetDevice(c->device);
    return hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream") &&
           hip_ok(hipMemcpy(sums, c->wsum_dump, (uint64_t)layers * 32 * 8, hipMemcpyDeviceToHost), err, err_len, "read");
}

int qxg_kv_read_position(qxg_ctx *c, uint32_t position, uint32_t layers, int8_t *k, int8_t *v, float *ks, float *vs,
                         char *err, uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!layers || layers > c->kv_layers || position >= c->kv_ctx || !k || !v || !ks || !vs) {
        set_err(err, err_len, "invalid argument");
        return 0;
    }
    (void)hipSetDevice(c->device);
    const uint64_t pitch = (uint64_t)c->kv_ctx * 512, spitch = (uint64_t)c->kv_ctx * 4;
    return hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream") &&
           hip_ok(hipMemcpy2D(k, 512, c->kc + (uint64_t)position * 512, pitch, 512, layers, hipMemcpyDeviceToHost), err, err_len, "read") &&
           hip_ok(hipMemcpy2D(v, 512, c->vc + (uint64_t)position * 512, pitch, 512, layers, hipMemcpyDeviceToHost), err, err_len, "read") &&
           hip_ok(hipMemcpy2D(ks, 4, c->ks + position, spitch, 4, layers, hipMemcpyDeviceToHost), err, err_len, "read") &&
           hip_ok(hipMemcpy2D(vs, 4, c->vs + position, spitch, 4, layers, hipMemcpyDeviceToHost), err, err_len, "read");
}

int qxg_set_attention_chunks(qxg_ctx *c, uint32_t min_positions) {
    if (!c) return 0;
    c->att_split_min = min_positions ? min_positions : 1u;
    return 1;
}

int qxg_set_layer_path(qxg_ctx *c, int persistent) {
    if (!c) return 0;
    if (c->persist != (persistent != 0)) {
        (void)hipSetDevice(c->device);
        if (c->s) (void)hipStreamSynchronize(c->s);
        drop_graph(c);
        c->persist = persistent != 0;
    }
    return 1;
}

int qxg_set_activation(qxg_ctx *c, uint32_t activation_format, char *err, uint64_t err_len) {
    if (!c) { set_err(err, err_len, "invalid context"); return 0; }
    if (activation_format > 1) { set_err(err, err_len, "unsupported activation format (0 f32, 1 q8_k_compat)"); return 0; }
    if (c->q8 != (activation_format == 1)) {
        (void)hipSetDevice(c->device);
        if (c->s) (void)hipStreamSynchronize(c->s);
        drop_graph(c);
        c->q8 = activation_format == 1;
    }
    return 1;
}

int qxg_prefill(qxg_ctx *c, const uint32_t *tokens, uint32_t n, uint32_t position0, int run_head, float *residual_out,
                float *logits, uint32_t top_n, uint32_t *top_ids, double *top_logits, float *elapsed_ms, char *err,
                uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!c->emb) { set_err(err, err_len, "token_embd.weight not bound"); return 0; }
    if (run_head && !c->head) { set_err(err, err_len, "head not bound"); return 0; }
    if (!tokens || !n) { set_err(err, err_len, "prefill needs >= 1 token"); return 0; }
    if ((uint64_t)position0 + n > c->kv_ctx || c->layers > c->kv_layers) { set_err(err, err_len, "prefill exceeds the KV context"); return 0; }
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= c->vocab) { set_err(err, err_len, "prompt token out of range"); return 0; }
    if (top_n == 0) top_n = 1;
    if (top_n > QXG_MAX_TOPN) top_n = QXG_MAX_TOPN;
    (void)hipSetDevice(c->device);
    c->kt.used = 0;
    if (!batched_prefill(c)) {
        if (persistent(c) && c->layers && !residual_out) {
            // the token steps in one persistent launch (the head on the last token only:
            // n_prompt one past the steps keeps it off), then the top-N of its logits
            if (!hip_ok(hipMemcpy(c->tokens, tokens, 4ull * n, hipMemcpyHostToDevice), err, err_len, "tokens")) return 0;
            write_state(c, position0, 0, n, run_head ? 1u : 0u);   // (force_head: the top-N kernels run after it)
            DecodeDumps d;
            d.logits = run_head ? c->logits : nullptr;
            d.norm = run_head ? c->norm : nullptr;
            (void)hipEventRecord(c->e0, c->s);
            if (!launch_decode(c, n, run_head ? n : n + 1, position0, false, d, err, err_len)) return 0;
            if (run_head) {
                hipLaunchKernelGGL(qxk_topk, dim3(TOPK_BLOCKS), dim3(256), 0, c->s, c->logits, c->vocab, top_n, c->cand_v,
                                   c->cand_i, c->top_v, c->top_i, c->tokens, c->st);
                hipLaunchKernelGGL(qxk_topk_merge, dim3(1), dim3(256), 0, c->s, (const float *)c->cand_v,
                                   (const uint32_t *)c->cand_i, (uint32_t)TOPK_BLOCKS, top_n, c->top_v, c->top_i, c->tokens, c->st);
            }
            (void)hipEventRecord(c->e1, c->s);
        } else if (!prefill_steps(c, tokens, n, position0, run_head, residual_out, top_n, err, err_len)) {
            return 0;
        }
        return prefill_finish(c, run_head, logits, top_n, top_ids, top_logits, elapsed_ms, err, err_len);
    }
    if (!prefill_ready(c, err, err_len)) return 0;
    auto &B = c->pf;
    if (!hip_ok(hipMemcpy(B.tokens, tokens, 4ull * (n < QXP_MAX ? n : QXP_MAX), hipMemcpyHostToDevice), err, err_len, "tokens"))
        return 0;
    (void)hipEventRecord(c->e0, c->s);
    for (uint32_t c0 = 0; c0 < n; c0 += QXP_MAX) {
        const uint32_t T = n - c0 < QXP_MAX ? n - c0 : QXP_MAX;
        if (c0) {   // earlier chunks are done with the token buffer once the stream reaches this copy
            if (!hip_ok(hipStreamSynchronize(c->s), err, err_len, "stream") ||
                !hip_ok(hipMemcpy(B.tokens, tokens + c0, 4ull * T, hipMemcpyHostToDevice), err, err_len, "tokens"))
                return 0;
        }
        hipLaunchKernelGGL(qxp_embed, dim3(T), dim3(256), 0, c->s, c->emb, c->emb_row, (const uint32_t *)B.tokens, B.X);
        for (uint32_t l = 0; l < c->layers; ++l) prefill_layer(c, l, T, position0 + c0, nullptr);
        if (residual_out &&
            !hip_ok(hipMemcpyAsync(residual_out + 2048ull * c0, B.X, 2048ull * 4 * T, hipMemcpyDeviceToHost, c->s), err, err_len, "read"))
            return 0;
        if (c0 + T == n && run_head) {
            (void)hipMemcpyAsync(c->x, B.X + 2048ull * (T - 1), 2048 * 4, hipMemcpyDeviceToDevice, c->s);
            write_state(c, position0 + n - 1, 0, 1, 1);
            launch_head(c, top_n, nullptr);
        }
    }
    (void)hipEventRecord(c->e1, c->s);
    return prefill_finish(c, run_head, logits, top_n, top_ids, top_logits, elapsed_ms, err, err_len);
}


int qxg_prefill_layer(qxg_ctx *c, uint32_t layer, uint32_t n, uint32_t position0, const float *x_in, float *ffn_inp_out,
                      float *moe_out, float *x_out, char *err, uint64_t err_len) {
    if (!check_ready(c, true, err, err_len)) return 0;
    if (!x_in || !n || n > QXP_MAX || layer >= c->layers || layer >= c->kv_layers || (uint64_t)position0 + n > c->kv_ctx) {
        set_err(err, err_len, "invalid prefill layer argument");
        return 0;
    }
    (void)hipSetDevice(c->device);
    c->kt.used = 0;
    if (!batched_prefill(c)) {   // token steps of the layer's attention and MoE halves
        for (uint32_t i = 0; i < n; ++i) {
            const uint64_t o = 2048ull * i;
            if (!hip_ok(hipMemcpyAsync(c->x, x_in + o, 2048 * 4, hipMemcpyHostToDevice, c->s), err, err_len, "upload")) return 0;
            write_state(c, position0 + i, 0, 1, 1);
            launch_attention(c, layer, c->x, nullptr, nullptr);
            if (ffn_inp_out && !hip_ok(hipMemcpyAsync(ffn_inp_out + o, c->x, 2048 * 4, hipMemcpyDeviceToHost, c->s), err, err_len, "read"))
                return 0;
            launch_moe(c, layer, c->x, c->moe);
            if ((moe_out && !hip_ok(hipMemcpyAsync(moe_out + o, c->moe, 2048 * 4, hipMemcpyDeviceToHost, c->s), err, err_len, "read")) ||
                (x_out && !hip_ok(hipMemcpyAsync(x_out + o, c->x, 2048 * 4, hipMemcpyDeviceToHost, c->s), err, err_len, "read")))
                return 0;
            if (!finish(c, err, err_len)) return 0;
        }
        return 1;
    }
    if (!prefill_ready(c, err, err_len)) return 0;
    auto &B = c->pf;
    if (!hip_ok(hipMemcpyAsync(B.X, x_in, 2048ull * 4 * n, hipMemcpyHostToDevice, c->s), err, err_len, "upload")) return 0;
    prefill_layer(c, layer, n, position0, moe_out ? B.dump : nullptr);
    if (!finish(c, err, err_len)) return 0;
    if (ffn_inp_out && !hip_ok(hipMemcpy(ffn_inp_out, B.X1, 2048ull * 4 * n, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (moe_out && !hip_ok(hipMemcpy(moe_out, B.dump, 2048ull * 4 * n, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    if (x_out && !hip_ok(hipMemcpy(x_out, B.X, 2048ull * 4 * n, hipMemcpyDeviceToHost), err, err_len, "read")) return 0;
    return 1;
}

/* In-situ timing of one kernel kind inside qxg_generate / qxg_decode_token:
 * an event pair is recorded around every launch of kernel `which` (numbering of
 * qxg_time_kernel; -1 disables). */
int qxg_profile_kernel(qxg_ctx *c, int which) {
    if (!c) return 0;
    c->kt.which = which;
    c->kt.used = 0;
    return 1;
}

int qxg_profile_result(qxg_ctx *c, uint32_t *launches, double *total_ms) {
    if (!c) return 0;
    double tot = 0.0;
    for (uint32_t i = 0; i < c->kt.used; ++i) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, c->kt.ev[2 * i], c->kt.ev[2 * i + 1]);
        tot += ms;
    }
    if (launches) *launches = c->kt.used;
    if (total_ms) *total_ms = tot;
    return 1;
}

}  // extern "C"
