// Persistent decode on gfx950: every step of a qxg_generate call (embedding, 48 layers,
// output head, argmax fed back) in one cooperative launch of one 512-thread workgroup per
// CU.  The layer loop body of the reference state loop (src/qx_format.c:6250-6627) runs as
// five stages per layer, handed over through epoch-tagged device words instead of kernel
// boundaries (a kernel boundary costs ~3.5 us on this GPU, a 2048-word all-to-all of
// tagged words ~1.8 us):
//   Q  attn RMSNorm + Q/K/V rows; router WGs: x-part of the router logits   (all WGs)
//   A  q/k norm, RoPE, INT8 K/V append, GQA softmax, context              (WG h = q head h)
//   O  O projection + residual; router WGs: ctx-part of the router logits (all WGs)
//   G  top-8, gate/up + SwiGLU; WG 0: renormalised expert weights         (all WGs)
//   D  down, rank-ordered weighted sum + residual                         (all WGs)
// then, on head steps, the output RMSNorm, the Q6_K head and the argmax.
//
// Router from the attention context.  The reference picks experts by the softmax of
// logit_e = sum_i W[e,i] * xn_i, xn = RMSNorm(x') with x' = x + O ctx
// (src/qx_format.c:5198-5290).  With w the ffn-norm weights and r = 1/rms(x'),
//     logit_e = r * (sum_i W[e,i] w_i x_i  +  sum_j M[e,j] ctx_j),   M = W diag(w) O,
// so the router needs only x (known in stage Q) and ctx (stage O's input), not x' - one
// all-to-all exchange fewer per layer.  r > 0 does not change the order, so the top-8 is
// taken from the bracket; the renormalised weights use r * bracket once x' is known.  M is
// formed once per model in double from the dequantized O rows and stored as f32
// (qxk_router_fold); the logits then differ from the reference's only by f32 roundings
// (~1e-7 relative), the router parity tests hold ids to the reference's with its 1e-4
// margin rule and the weights to 1e-6.
//
// Exchanges.  A word is {epoch:32, payload:32}, written and read with relaxed agent-scope
// atomics (single-copy atomic, coherent across XCDs without cache maintenance): a consumer
// polls until every word it needs carries the epoch of the current phase.  Each buffer has
// two slots (layer parity); every layer passes an all-to-all dependency through every
// workgroup, so no workgroup is ever two layers ahead of another and a slot is never
// overwritten while still being read.  Every wait is bounded by a deadline and a shared
// abort flag, so all waves exit even if a producer never arrives.
//
// Weight prefetch.  A wave's loads complete in issue order, so a poll issued behind
// outstanding weight loads waits for them; weight loads are therefore issued right after
// a poll completes, for a stage at least one exchange later: the next layer's Q/K/V rows
// after this layer's Q stage (after the attention stage in attention workgroups), the
// next layer's O rows, router rows and norm weights after stage G, the routed experts'
// gate/up and down rows right after the top-8.
#include "qxg_dev.h"

// Stage timestamps for development builds only (-DQXD_TRACE): on the last step, lane 0 of
// each workgroup's wave 0 stores s_memrealtime (100 MHz) into
// qxd_trace_buf[layer][point][workgroup]; read back with qxd_trace_read.
#ifdef QXD_TRACE
__device__ unsigned long long qxd_trace_buf[49][24][256];
extern "C" int qxd_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(qxd_trace_buf), sizeof(qxd_trace_buf)) == hipSuccess;
}
#define DMARK(layer, point)                                                                                   \
    do {                                                                                                      \
        if (last && (threadIdx.x == 0)) qxd_trace_buf[layer][point][blockIdx.x] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define DMARK(layer, point) ((void)0)
#endif

namespace {

constexpr int NT = 512;            // threads per workgroup
constexpr int NWV = NT / 64;       // waves per workgroup
constexpr int NWG = QXG_PBLOCKS;   // workgroups, one per CU

// exchange buffers: word offsets of slot 0 (slot 1 follows at + size)
constexpr uint32_t XN_X = 2048, XN_QKV = 5120, XN_CX = 4096, XN_XP = 2048, XN_LG = 256, XN_H = 6144, XN_WT = 16,
                   XN_AM = 2 * NWG;
constexpr uint32_t XO_X = 0;
constexpr uint32_t XO_QKV = XO_X + 2 * XN_X;
constexpr uint32_t XO_CX = XO_QKV + 2 * XN_QKV;
constexpr uint32_t XO_XP = XO_CX + 2 * XN_CX;
constexpr uint32_t XO_LG = XO_XP + 2 * XN_XP;
constexpr uint32_t XO_H = XO_LG + 2 * XN_LG;
constexpr uint32_t XO_WT = XO_H + 2 * XN_H;
constexpr uint32_t XO_AM = XO_WT + 2 * XN_WT;
constexpr uint32_t XO_END = XO_AM + 2 * XN_AM;

#define GLB __attribute__((address_space(1)))
DEV uint64_t xld(const GLB uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void xst(GLB uint64_t *p, uint32_t ep, uint32_t bits) {
    __hip_atomic_store(p, ((uint64_t)ep << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void xstf(GLB uint64_t *p, uint32_t ep, float v) { xst(p, ep, __float_as_uint(v)); }
DEV void st_coherent(GLB uint32_t *p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV uint32_t ld_coherent(const GLB uint32_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// The thread index as a value the compiler cannot hoist: each stage derives its lane
// indices from its own copy, so they are recomputed where used (a few ALU ops) instead of
// being held, or spilled, across the whole persistent loop.
DEV int tix() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

struct Ctl {
    GLB uint32_t *abort;
    uint64_t timeout;
};

// true while a wait may go on; every 64 polls checks its deadline and the abort flag
DEV bool keep_waiting(uint32_t &it, uint64_t deadline, const Ctl &c) {
    if ((++it & 63u) != 0) return true;
    if (wall_clock64() > deadline || __hip_atomic_load(c.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
        __hip_atomic_store(c.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return true;
}

// Waits until words idx(i), i < n, all carry epoch ep and stores their payloads to dst[i];
// threads 0 .. P-1 take words tid, tid + P, ... (K >= n / P each).  Reloads only stale
// words.  Returns false on timeout/abort; the caller makes that block-uniform.
template <int K, int P = 512, typename IDX>
DEV bool poll(const GLB uint64_t *base, int n, uint32_t ep, uint32_t *dst, IDX idx, const Ctl &c) {
    const int tid = tix();
    constexpr int NT = P;
    uint64_t w[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = tid + NT * k;
        w[k] = i < n ? xld(base + idx(i)) : ((uint64_t)ep << 32);
    }
    const uint64_t deadline = wall_clock64() + c.timeout;
    uint32_t it = 0;
    bool ok = true;
    for (;;) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < K; ++k) all = all && (uint32_t)(w[k] >> 32) == ep;
        if (all) break;
        if (!keep_waiting(it, deadline, c)) { ok = false; break; }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = tid + NT * k;
            if (i < n && (uint32_t)(w[k] >> 32) != ep) w[k] = xld(base + idx(i));
        }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = tid + NT * k;
        if (i < n) dst[i] = (uint32_t)w[k];
    }
    return ok;
}
struct Ident {
    DEV int operator()(int i) const { return i; }
};

// Wave-uniform pointer arithmetic on the arguments (scalar registers).
DEV uint64_t uni64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

}  // namespace

static_assert(XO_END == QXD_XCH_WORDS, "exchange layout");
static_assert(NT == QXD_THREADS, "workgroup size");

namespace {

// ---------------------------------------------------------------- LDS
struct AttnS {
    float q[128], k[512], v[512];
    uint32_t qd[4 * DIG_STRIDE];
    int8_t kq[512], vq[512];     // the position's INT8 K and V rows (all four kv heads)
    double sc[QXG_MAX_CTX];      // scores, then weights
    float part[32][132];         // context partial sums
    float mx[2 * NWV];
    double redd[2 * NWV];
    float scale[2];
};
struct DLds {
    uint4 g2[512];
    uint2 g3[256];
    uint2 sel[128];
    float xs[2048];              // layer input x (stage Q .. O residual)
    float xp[2048];              // x' = x + O ctx (stage G .. D residual)
    uint32_t dig[192 * DIG_STRIDE];
    double red[2 * NWV];
    uint32_t lgw[2 * 128];       // router logits (hi, lo words)
    float outw[32];              // the workgroup's outputs of a stage, gathered for one store
    uint32_t flag[NWV];
    union {
        uint32_t vin[6144 + 16]; // polled ctx (4096), or h (6144) and the 8 expert weights
        AttnS att;
        struct {
            float bv[NWV];
            uint32_t bi[NWV];
            uint32_t am[XN_AM];
        } hd;
    } u;
};

// block-wide OR of a per-thread flag (every thread of the workgroup calls it); includes
// the barrier that publishes the caller's earlier LDS writes
DEV bool block_any(bool f, DLds &S) {
    const bool any = __ballot(f) != 0;
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) S.flag[wave] = any ? 1u : 0u;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) r |= S.flag[w];
    return r != 0;
}

// A workgroup's wait for an exchange.  Producers publish each workgroup's words with one
// store instruction, so the first word of every producer's block (its sentinel) is polled
// alone while the producers finish - a few KB per round instead of the whole vector - and
// only then every word is read, words not yet carrying the epoch being read again.  All
// threads call it; the payloads are in dst (LDS) when it returns true.  sidx(j) < nsent:
// word offsets of the sentinels; idx(i) < n: of the payload words (both from base).
// EARLY: the words are read once first (one round trip when they are already there, as for
// exchanges whose producers finished well before the wait); only if some are stale does
// the sentinel phase follow.
template <int K, bool EARLY = false, typename IDX, typename SIDX>
DEV bool wait_xch(const GLB uint64_t *base, int n, uint32_t ep, uint32_t *dst, IDX idx, int nsent, SIDX sidx, DLds &S,
                  const Ctl &c) {
    const int tid = tix();
    bool ok = true;
    if constexpr (EARLY) {
        bool have = true;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = tid + NT * k;
            if (i < n) {
                const uint64_t w = xld(base + idx(i));
                have = have && (uint32_t)(w >> 32) == ep;
                dst[i] = (uint32_t)w;
            }
        }
        if (!block_any(!have, S)) return true;
    }
    for (int j = tid; j < nsent; j += NT) {
        const GLB uint64_t *p = base + sidx(j);
        uint64_t w = xld(p);
        const uint64_t deadline = wall_clock64() + c.timeout;
        uint32_t it = 0;
        while ((uint32_t)(w >> 32) != ep) {
            if (!keep_waiting(it, deadline, c)) { ok = false; break; }
            w = xld(p);
        }
        if (!ok) break;
    }
    if (block_any(!ok, S)) return false;
    ok = poll<K>(base, n, ep, dst, idx, c);
    return !block_any(!ok, S);
}

// Digit planes of an N-vector held in LDS (as f32 bits), 8 values per thread-chunk; with
// NORM it is first RMS-normalised (reference src/qx_format.c:3358-3371), w8 the norm
// weights of the thread's 8 values (threads < 256).
// The inverse RMS goes to *inv_out.  Returns true when every value is finite.
template <int N, bool NORM>
DEV bool vec_digits(const float *v, const float *w8, DLds &S, double *inv_out = nullptr) {
    constexpr int NCH = N / 8;
    const int tid = tix(), lane = tid & 63, wave = tid >> 6;
    double inv = 1.0;
    if constexpr (NORM) {
        static_assert(N == 2048, "normalised vectors are 2048 long");
        double ss = 0.0;
        if (tid < 256) {
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += (double)v[8 * tid + i] * (double)v[8 * tid + i];
        }
        ss = wave_total_d(ss);
        if (lane == 0) S.red[wave] = ss;
        __syncthreads();
        const double tot = (S.red[0] + S.red[1]) + (S.red[2] + S.red[3]);   // waves 4..7 hold no values
        inv = 1.0 / sqrt(tot / 2048.0 + 1.0e-6);
        if (inv_out) *inv_out = inv;
    }
    bool fin = true;
    for (int c = tid; c < NCH; c += NT) {   // whole quads (a group) take the same branch
        float y[8];
        const float4 a = *reinterpret_cast<const float4 *>(v + 8 * c), b = *reinterpret_cast<const float4 *>(v + 8 * c + 4);
        y[0] = a.x; y[1] = a.y; y[2] = a.z; y[3] = a.w; y[4] = b.x; y[5] = b.y; y[6] = b.z; y[7] = b.w;
        if constexpr (NORM) {   // c == tid: w8 holds the thread's 8 weights
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = (float)((double)y[i] * inv) * w8[i];
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) { fin = fin && isfinite(y[i]); mx = fmaxf(mx, fabsf(y[i])); }
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
        uint32_t h0, h1, m0, m1, l0, l1;
        float sc;
        digits8(y, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
        uint32_t *d = S.dig + (c >> 2) * DIG_STRIDE;
        const int q = c & 3;
        *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
        *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
        *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
        if (q == 0) d[24] = __float_as_uint(sc);
    }
    return !block_any(!fin, S);
}

// Global-memory views: a uniform base in scalar registers plus a 32-bit per-lane offset
// (global_load v, v_off, s[base]); weight bytes with non-temporal loads, F32 rows cached.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <typename T>
DEV const GLB T *gp(const T *p) { return (const GLB T *)uni64((uint64_t)p); }
template <typename T>
DEV GLB T *gpw(T *p) { return (GLB T *)uni64((uint64_t)p); }
DEV uint4 gnt4(const GLB uint8_t *b, uint32_t off) {
    const u32x4 v = __builtin_nontemporal_load((const GLB u32x4 *)(b + off));
    return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint2 gnt2(const GLB uint8_t *b, uint32_t off) {
    const u32x2 v = __builtin_nontemporal_load((const GLB u32x2 *)(b + off));
    return make_uint2(v.x, v.y);
}
DEV uint32_t gnt1(const GLB uint8_t *b, uint32_t off) { return __builtin_nontemporal_load((const GLB uint32_t *)(b + off)); }
DEV float4 ldf4(const GLB uint8_t *b, uint32_t off) {
    const f32x4 v = *(const GLB f32x4 *)(b + off);
    return make_float4(v.x, v.y, v.z, v.w);
}

// layer l's plane `id` (scalar arithmetic on the argument copy)
DEV const GLB uint8_t *plane(const QxDArgs &a, int id, uint32_t l) {
    return (const GLB uint8_t *)(uni64((uint64_t)a.P[id].base) + (uint64_t)l * uni64(a.P[id].stride));
}

// ---------------------------------------------------------------- weight sets
// Q/K/V rows of a wave: Q rows 16 wg + 2 w + {0, 1}; waves 0..3 also K/V row 4096 + 4 wg + w
// (waves 4..7 load their partner's, unused), and the attn-norm weights of the thread's 8
// values.  Every load is unconditional: a register set reloaded on every path is not kept
// live across the stages in between.
struct WQ {
    uint4 q[3];
    uint2 m[3];
    float4 nw0, nw1;
};
DEV void load_wq(const QxDArgs &a, uint32_t l, WQ &w) {
    const int tid = tix(), lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
    const uint32_t b = lane >> 3, ib = lane & 7;
    const GLB uint8_t *qq = plane(a, PL_Q_QS, l), *qm = plane(a, PL_Q_META, l);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t blk = (uint32_t)(16 * wg + 2 * wave + r) * 8 + b;
        w.q[r] = gnt4(qq, blk * 128 + 16 * ib);
        w.m[r] = gnt2(qm, blk * 8);
    }
    const uint32_t kv = 4 * wg + (wave & 3);   // 0..1023: K rows 0..511, then V rows
    const GLB uint8_t *kq = kv < 512 ? plane(a, PL_K_QS, l) : plane(a, PL_V_QS, l);
    const GLB uint8_t *km = kv < 512 ? plane(a, PL_K_META, l) : plane(a, PL_V_META, l);
    const uint32_t blk = (kv & 511) * 8 + b;
    w.q[2] = gnt4(kq, blk * 128 + 16 * ib);
    w.m[2] = gnt2(km, blk * 8);
    const GLB uint8_t *nw = plane(a, PL_ATTN_NORM, l);
    w.nw0 = ldf4(nw, 32 * (tid & 255));
    w.nw1 = ldf4(nw, 32 * (tid & 255) + 16);
}
// O row 8 wg + w (16 blocks; lane takes blocks lane/8 and 8 + lane/8, sub-block lane%8)
// and router row W[e] with the ffn-norm weights, values 4 tid .. 4 tid + 3 (the router's
// x-part; workgroups e >= experts load an unused copy)
struct WO {
    uint4 q0, q1;
    uint2 m0, m1;
    float4 wr, fw;
};
DEV void load_wo(const QxDArgs &a, uint32_t l, WO &w) {
    const int tid = tix(), lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
    const uint32_t ib = lane & 7;
    const GLB uint8_t *oq = plane(a, PL_O_QS, l), *om = plane(a, PL_O_META, l);
    const uint32_t r = (uint32_t)(8 * wg + wave) * 16;
    const uint32_t k0 = r + (lane >> 3), k1 = r + 8 + (lane >> 3);
    w.q0 = gnt4(oq, k0 * 128 + 16 * ib);
    w.q1 = gnt4(oq, k1 * 128 + 16 * ib);
    w.m0 = gnt2(om, k0 * 8);
    w.m1 = gnt2(om, k1 * 8);
    const uint32_t e = min((uint32_t)wg, a.experts - 1);
    w.wr = ldf4(plane(a, PL_ROUTER, l), e * 8192 + 16 * tid);
    w.fw = ldf4(plane(a, PL_FFN_NORM, l), 16 * tid);
}
// router fold row M[e], values 8 tid .. 8 tid + 7 (the router's ctx-part)
DEV void load_wm(const QxDArgs &a, uint32_t l, float4 &m0, float4 &m1) {
    const int tid = tix(), wg = blockIdx.x;
    const uint32_t e = min((uint32_t)wg, a.experts - 1);
    const GLB uint8_t *mm = (const GLB uint8_t *)(uni64((uint64_t)a.M.base) + (uint64_t)l * uni64(a.M.stride));
    m0 = ldf4(mm, e * 16384 + 32 * tid);
    m1 = ldf4(mm, e * 16384 + 32 * tid + 16);
}
// norm weights of the thread's 8 values 8 tid .. 8 tid + 7 (used by threads < 256; the
// others load a copy)
DEV void load_w8(const GLB uint8_t *p, float (&w)[8]) {
    const uint32_t t = tix() & 255;
    const float4 x0 = ldf4(p, 32 * t), x1 = ldf4(p, 32 * t + 16);
    w[0] = x0.x; w[1] = x0.y; w[2] = x0.z; w[3] = x0.w;
    w[4] = x1.x; w[5] = x1.y; w[6] = x1.z; w[7] = x1.w;
}
// routed experts' rows of a wave: gate/up units 3 gw .. 3 gw + 2 (one expert per wave:
// 768 = 256 * 3); down row 8 wg + w of all 8 ranks (lane 8 r + k: rank r, sub-block k of
// the 3 blocks)
struct WE {
    uint2 gq[3], uq[3];
    uint32_t gs[3], us[3], gd[3], ud[3];
};
struct WD {
    uint2 dq[3];
    uint32_t dax[3], dd[3];
};
DEV uint32_t ld_u8(const GLB uint8_t *b, uint32_t off) { return b[off]; }
DEV uint32_t ld_u16(const GLB uint8_t *b, uint32_t off) { return *(const GLB uint16_t *)(b + off); }
DEV void load_we(const QxDArgs &a, uint32_t l, const uint32_t (&ids)[QXG_TOPK], WE &w) {
    const int tid = tix(), lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
    const uint32_t b = lane >> 3, ib = lane & 7;
    const int u0 = 3 * (NWV * wg + wave);
    uint32_t e = 0u;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q)
        if (q == u0 / QXG_FFN) e = ids[q];
    const GLB uint8_t *gqs = plane(a, PL_G_QS, l), *gsc = plane(a, PL_G_SC, l), *gdd = plane(a, PL_G_D, l);
    const GLB uint8_t *uqs = plane(a, PL_U_QS, l), *usc = plane(a, PL_U_SC, l), *udd = plane(a, PL_U_D, l);
#pragma unroll
    for (int uu = 0; uu < 3; ++uu) {
        const uint32_t blk = (e * QXG_FFN + (uint32_t)((u0 + uu) % QXG_FFN)) * 8 + b;
        w.gq[uu] = gnt2(gqs, blk * 64 + 8 * ib);
        w.uq[uu] = gnt2(uqs, blk * 64 + 8 * ib);
        w.gs[uu] = ld_u8(gsc, blk * 8 + ib);
        w.us[uu] = ld_u8(usc, blk * 8 + ib);
        w.gd[uu] = ld_u16(gdd, blk * 2);
        w.ud[uu] = ld_u16(udd, blk * 2);
    }
}
DEV void load_wd(const QxDArgs &a, uint32_t l, const uint32_t (&ids)[QXG_TOPK], WD &w) {
    const int tid = tix(), lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
    const uint32_t r = lane >> 3, k = lane & 7;
    uint32_t de = 0u;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q)
        if (q == (int)r) de = ids[q];
    const GLB uint8_t *dqs = plane(a, PL_D_QS, l), *dax = plane(a, PL_D_AUX, l), *ddd = plane(a, PL_D_D, l);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const uint32_t blk = (de * 2048 + 8 * wg + wave) * 3 + j;
        w.dq[j] = gnt2(dqs, blk * 64 + 8 * k);
        w.dax[j] = gnt1(dax, blk * 32 + 4 * k);
        w.dd[j] = ld_u16(ddd, blk * 2);
    }
}

// ---------------------------------------------------------------- attention (stage A)
// Workgroup h: q head h (reference qx_rope_gqa_attention_partial, src/qx_format.c:5051-5196,
// and the state loop's K/V handling, 6282-6363): per-head q/k RMSNorm (3740-3757), RoPE
// (4625-4641, host table), INT8 K/V quantization of the position over all 512 values
// (4449-4463; workgroup 0 stores the rows, every workgroup derives the same row), scores of
// q as int8 digit planes against the INT8 K codes (v_dot4, exact), double softmax, f32
// context.  Rows of positions written by this launch (>= pos0) are read with coherent
// loads, older rows with plain loads.
//
// The cached rows of the first ATT_PRE positions are fetched before the Q/K/V exchange is
// polled (their addresses depend only on the layer and the position count): thread t
// takes the 32 K bytes of group t%4 of position t/4 (the score loop's first pass) and the
// 8 V bytes of dims 8(t%16).. of positions t/16 + 32 i (the context loop's).
constexpr uint32_t ATT_PRE = 128;
struct AttnPre {   // vector-typed fields: they stay in registers (arrays filled in branches did not)
    u32x4 k0, k1;
    float ks;
    u32x2 v0, v1, v2, v3;
    float vs;          // V scale of position tid (the softmax loop's first pass)
    double cs, sn;     // RoPE table entries of the position, dims lane and lane + 64
    float n0, n1;      // k-norm weights (waves 0..3) or q-norm weights (wave 4), dims lane, lane + 64
};
DEV void attn_prefetch(const QxDArgs &a, uint32_t l, uint32_t pos, AttnPre &p) {
    const int tid = tix();
    const int kvh = blockIdx.x >> 3;
    const GLB uint32_t *kc = (const GLB uint32_t *)gp(a.kc), *vc = (const GLB uint32_t *)gp(a.vc);
    const GLB uint32_t *ksw = (const GLB uint32_t *)gp(a.ks);
    const uint32_t base = l * a.ctx, fresh = a.pos0;
    {   // K: position tid/4 (clamped: positions past pos - 1 are never used)
        const uint32_t t = min((uint32_t)tid >> 2, pos > 0 ? pos - 1 : 0u);
        const GLB uint32_t *kp = kc + (base + t) * 128 + 32 * kvh + 8 * (tid & 3);
        if (t >= fresh) {
            p.k0 = u32x4{ld_coherent(kp), ld_coherent(kp + 1), ld_coherent(kp + 2), ld_coherent(kp + 3)};
            p.k1 = u32x4{ld_coherent(kp + 4), ld_coherent(kp + 5), ld_coherent(kp + 6), ld_coherent(kp + 7)};
            p.ks = __uint_as_float(ld_coherent(ksw + base + t));
        } else {
            p.k0 = *(const GLB u32x4 *)kp;
            p.k1 = *(const GLB u32x4 *)(kp + 4);
            p.ks = __uint_as_float(ksw[base + t]);
        }
    }
    // V: positions tid/16 + 32 i
    auto vld = [&](uint32_t i) -> u32x2 {
        const uint32_t t = min((uint32_t)(tid >> 4) + 32u * i, pos > 0 ? pos - 1 : 0u);
        const GLB uint32_t *vp = vc + (base + t) * 128 + 32 * kvh + 2 * (tid & 15);
        if (t >= fresh) return u32x2{ld_coherent(vp), ld_coherent(vp + 1)};
        return *(const GLB u32x2 *)vp;
    };
    p.v0 = vld(0); p.v1 = vld(1); p.v2 = vld(2); p.v3 = vld(3);
    {
        const GLB uint32_t *vsw = (const GLB uint32_t *)gp(a.vs);
        const uint32_t t = min((uint32_t)tid, pos > 0 ? pos - 1 : 0u);
        p.vs = __uint_as_float(t >= fresh ? ld_coherent(vsw + base + t) : vsw[base + t]);
    }
    const int lane = tid & 63;
    p.cs = gp(a.T.rope_cos)[pos * 64 + lane];
    p.sn = gp(a.T.rope_sin)[pos * 64 + lane];
    const GLB float *nw = (const GLB float *)plane(a, (tid >> 6) == 4 ? PL_Q_NORM : PL_K_NORM, l);
    p.n0 = nw[lane];
    p.n1 = nw[64 + lane];
}

// The Q/K/V words of head h's workgroup: q rows 128 h .. 128 h + 127, then the K and V rows
// (4096 .. 5119), into A.q, A.k, A.v; sentinels: the K/V word of each producer workgroup
// (published with its Q rows in one store)
DEV bool attn_wait(const QxDArgs &a, uint32_t l, uint32_t ep, DLds &S, const Ctl &c) {
    const int h = blockIdx.x;
    const GLB uint64_t *qkv = gp(a.xch) + XO_QKV + (l & 1) * XN_QKV;
    return wait_xch<3>(qkv, 1152, ep, reinterpret_cast<uint32_t *>(S.u.att.q),
                       [h](int i) { return i < 128 ? 128 * h + i : 3968 + i; }, NWG, [](int j) { return 4096 + 4 * j; }, S, c);
}

// ep: the QKV phase (the context goes out at ep + 1)
DEV void attention(const QxDArgs &a, uint32_t l, uint32_t pos, uint32_t ep, const AttnPre &pre, DLds &S) {
    AttnS &A = S.u.att;
    const int tid = tix(), lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, kvh = h >> 3;
    const uint32_t n = pos + 1;
    const double cs = pre.cs, sn = pre.sn;
    if (wave < 4) {   // k of kv head `wave`
        float k0 = A.k[128 * wave + lane], k1 = A.k[128 * wave + 64 + lane];
        head_norm_rope_wave(k0, k1, pre.n0, pre.n1, cs, sn);
        A.k[128 * wave + lane] = k0;
        A.k[128 * wave + 64 + lane] = k1;
    } else if (wave == 4) {
        float q0 = A.q[lane], q1 = A.q[64 + lane];
        head_norm_rope_wave(q0, q1, pre.n0, pre.n1, cs, sn);
        A.q[lane] = q0;
        A.q[64 + lane] = q1;
    }
    __syncthreads();
    // INT8 K/V rows: scale = max|x| / 127 (1 if zero), codes rint(x / scale) clamped
    float ka = isfinite(A.k[tid]) ? fabsf(A.k[tid]) : 0.0f, va = isfinite(A.v[tid]) ? fabsf(A.v[tid]) : 0.0f;
    ka = fmaxf(ka, dppf<DPP_XOR1>(ka)); va = fmaxf(va, dppf<DPP_XOR1>(va));
    ka = fmaxf(ka, dppf<DPP_XOR2>(ka)); va = fmaxf(va, dppf<DPP_XOR2>(va));
    ka = fmaxf(ka, dppf<DPP_ROR4>(ka)); va = fmaxf(va, dppf<DPP_ROR4>(va));
    ka = fmaxf(ka, dppf<DPP_ROR8>(ka)); va = fmaxf(va, dppf<DPP_ROR8>(va));
    ka = fmaxf(fmaxf(rdlanef(ka, 0), rdlanef(ka, 16)), fmaxf(rdlanef(ka, 32), rdlanef(ka, 48)));
    va = fmaxf(fmaxf(rdlanef(va, 0), rdlanef(va, 16)), fmaxf(rdlanef(va, 32), rdlanef(va, 48)));
    if (lane == 0) { A.mx[wave] = ka; A.mx[NWV + wave] = va; }
    // q digit planes (4 groups of 32: threads 0..15, 8 values each, quads share a group)
    bool qfin = true;
    if (tid < 16) {
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { y[i] = A.q[8 * tid + i]; qfin = qfin && isfinite(y[i]); }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(y[i]));
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
        uint32_t h0, h1, m0, m1, l0, l1;
        float scq;
        digits8(y, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, scq);
        uint32_t *d = A.qd + (tid >> 2) * DIG_STRIDE;
        const int q = tid & 3;
        *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
        *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
        *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
        if (q == 0) d[24] = __float_as_uint(scq);
    }
    const bool qok = !block_any(!qfin, S);   // barrier: A.mx, A.qd visible
    float kmx = 0.0f, vmx = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) { kmx = fmaxf(kmx, A.mx[w]); vmx = fmaxf(vmx, A.mx[NWV + w]); }
    const float kscale = kmx > 0.0f ? kmx / 127.0f : 1.0f, vscale = vmx > 0.0f ? vmx / 127.0f : 1.0f;
    {
        const float kx = A.k[tid], vx = A.v[tid];
        int qk = isfinite(kx) ? (int)rintf(kx / kscale) : 0;
        int qv = isfinite(vx) ? (int)rintf(vx / vscale) : 0;
        A.kq[tid] = (int8_t)(qk < -127 ? -127 : qk > 127 ? 127 : qk);
        A.vq[tid] = (int8_t)(qv < -127 ? -127 : qv > 127 ? 127 : qv);
    }
    __syncthreads();
    // the cache as 32-bit words: rows of 128 words, scales at [layer * ctx + position]
    GLB uint32_t *kc = (GLB uint32_t *)gpw(a.kc), *vc = (GLB uint32_t *)gpw(a.vc);
    GLB uint32_t *ksw = (GLB uint32_t *)gpw(a.ks), *vsw = (GLB uint32_t *)gpw(a.vs);
    const uint32_t base = l * a.ctx;   // slot of position 0 (layers * ctx * 512 < 2^32)
    if (h == 0) {   // the position's rows into the cache, coherent (later steps read them)
        const uint32_t slot = base + pos;
        if (tid < 128) st_coherent(kc + slot * 128 + tid, reinterpret_cast<const uint32_t *>(A.kq)[tid]);
        else if (tid < 256) st_coherent(vc + slot * 128 + (tid - 128), reinterpret_cast<const uint32_t *>(A.vq)[tid - 128]);
        else if (tid == 256) st_coherent(ksw + slot, __float_as_uint(kscale));
        else if (tid == 257) st_coherent(vsw + slot, __float_as_uint(vscale));
    }
    // scores: a quad per position, lane q4 the 32-dim group q4 of kv head kvh
    const int q4 = tid & 3;
    Dig d;
    load_dig(A.qd, q4, d);
    double mx = -1.0e300;
    const uint32_t fresh = a.pos0;   // rows >= fresh were written by this launch
    for (uint32_t t = tid >> 2; t < n; t += NT / 4) {
        uint32_t kw[8];
        float ksc;
        if (t == pos) {
            const uint4 *p = reinterpret_cast<const uint4 *>(A.kq + 128 * kvh + 32 * q4);
            const uint4 x0 = p[0], x1 = p[1];
            kw[0] = x0.x; kw[1] = x0.y; kw[2] = x0.z; kw[3] = x0.w; kw[4] = x1.x; kw[5] = x1.y; kw[6] = x1.z; kw[7] = x1.w;
            ksc = kscale;
        } else if (t < ATT_PRE) {   // t = tid / 4: the prefetched row
            kw[0] = pre.k0.x; kw[1] = pre.k0.y; kw[2] = pre.k0.z; kw[3] = pre.k0.w;
            kw[4] = pre.k1.x; kw[5] = pre.k1.y; kw[6] = pre.k1.z; kw[7] = pre.k1.w;
            ksc = pre.ks;
        } else {
            const GLB uint32_t *p = kc + (base + t) * 128 + 32 * kvh + 8 * q4;
            if (t >= fresh) {
#pragma unroll
                for (int i = 0; i < 8; ++i) kw[i] = ld_coherent(p + i);
                ksc = __uint_as_float(ld_coherent(ksw + base + t));
            } else {
                const u32x4 x0 = *(const GLB u32x4 *)p, x1 = *(const GLB u32x4 *)(p + 4);
                kw[0] = x0.x; kw[1] = x0.y; kw[2] = x0.z; kw[3] = x0.w; kw[4] = x1.x; kw[5] = x1.y; kw[6] = x1.z; kw[7] = x1.w;
                ksc = __uint_as_float(ksw[base + t]);
            }
        }
        int aH = 0, aM = 0, aL = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            aH = sdot4(kw[i], d.h[i], aH);
            aM = sdot4(kw[i], d.m[i], aM);
            aL = sdot4(kw[i], d.l[i], aL);
        }
        double acc = (double)(combine(aH, aM, aL) * d.s);
        acc += dppd<DPP_XOR1>(acc);
        acc += dppd<DPP_XOR2>(acc);
        double sc = qok ? acc * (double)ksc / a.sqrt_hd : 0.0;
        if (!isfinite(sc)) sc = 0.0;
        if (q4 == 0) A.sc[t] = sc;
        mx = fmax(mx, sc);
    }
    mx = wave_max_d(mx);
    if (lane == 0) A.redd[wave] = mx;
    __syncthreads();
    mx = A.redd[0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) mx = fmax(mx, A.redd[w]);
    // softmax in double: e_t = exp(s_t - mx), den = sum e_t (1 if not finite and positive)
    double den = 0.0;
    for (uint32_t t = tid; t < n; t += NT) {
        const double e = exp(A.sc[t] - mx);
        A.sc[t] = e;
        den += e;
    }
    den = wave_total_d(den);
    if (lane == 0) A.redd[NWV + wave] = den;
    __syncthreads();
    den = ((A.redd[NWV + 0] + A.redd[NWV + 1]) + (A.redd[NWV + 2] + A.redd[NWV + 3])) +
          ((A.redd[NWV + 4] + A.redd[NWV + 5]) + (A.redd[NWV + 6] + A.redd[NWV + 7]));
    if (!isfinite(den) || den <= 0.0) den = 1.0;
    // weights with the V scales folded in
    for (uint32_t t = tid; t < n; t += NT) {
        float vsc;
        if (t == pos) vsc = vscale;
        else if (t < NT) vsc = pre.vs;   // t = tid: prefetched
        else if (t >= fresh) vsc = __uint_as_float(ld_coherent(vsw + base + t));
        else vsc = __uint_as_float(vsw[base + t]);
        A.sc[t] = (A.sc[t] / den) * (double)vsc;
    }
    __syncthreads();
    // context: thread (g = tid / 16, 8 dims 8 (tid % 16) ..) sums positions g, g + 32, ...;
    // the 32 partial sums of a dimension are added in g order
    {
        const int g = tid >> 4, dg = tid & 15;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        uint32_t i = 0;
        for (uint32_t t = g; t < n; t += 32, ++i) {
            const float p = (float)A.sc[t];
            uint32_t v0, v1;
            if (t == pos) {
                const uint2 x = reinterpret_cast<const uint2 *>(A.vq + 128 * kvh)[dg];
                v0 = x.x; v1 = x.y;
            } else if (t < ATT_PRE) {   // t = tid / 16 + 32 i: the prefetched row
                const u32x2 x = i == 0 ? pre.v0 : i == 1 ? pre.v1 : i == 2 ? pre.v2 : pre.v3;
                v0 = x.x; v1 = x.y;
            } else {
                const GLB uint32_t *vp = vc + (base + t) * 128 + 32 * kvh + 2 * dg;
                if (t >= fresh) { v0 = ld_coherent(vp); v1 = ld_coherent(vp + 1); }
                else { const u32x2 x = *(const GLB u32x2 *)vp; v0 = x.x; v1 = x.y; }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int8_t vb = (int8_t)((((j < 4) ? v0 : v1) >> (8 * (j & 3))) & 255u);
                acc[j] = fmaf(p, (float)vb, acc[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) A.part[g][8 * dg + j] = acc[j];
    }
    __syncthreads();
    if (tid < 128) {
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) o += A.part[i][tid];
        xstf(gpw(a.xch) + XO_CX + (l & 1) * XN_CX + 128 * h + tid, ep + 1, o);   // the CX phase
    }
    __syncthreads();   // the union is reused by the next stage
}

// ---------------------------------------------------------------- head
// Output RMSNorm + Q6_K head (src/qx_format.c:3554-3738) over the digits in S.dig: wave
// gw takes rows R gw .. R gw + R - 1, then R (gw + 2048) .., R rows' loads in flight at a
// time; returns the workgroup's best (logit desc, index asc) through bv/bi (uniform);
// non-finite logits set *nonfin.
template <int R>
DEV void head_rows(const QxDArgs &a, DLds &S, bool fin, float &bv, uint32_t &bi, bool &nonfin) {
    const int tid = tix(), lane = tid & 63, wave = tid >> 6;
    const int b = lane >> 3, ib = lane & 7, hh = ib >> 2, k = ib & 3;
    const int gw = NWV * blockIdx.x + wave;
    Dig g;
    load_dig(S.dig, lane, g);
    const Q6Bias bias = q6_bias(g);
    float best = -INFINITY;
    uint32_t besti = 0xffffffffu;
    bool nf = false;
    const uint32_t groups = (a.vocab + R - 1) / R;
    const GLB uint8_t *hql = gp(a.h_ql), *hqh = gp(a.h_qh), *hsc = gp((const uint8_t *)a.h_sc), *hd = gp((const uint8_t *)a.h_d);
    GLB float *lg = a.logits ? gpw(a.logits) : nullptr;
    for (uint32_t p = gw; p < groups; p += NWV * NWG) {
        uint4 l0[R], l1[R], h0[R], h1[R];
        int s0[R], s1[R];
        uint32_t d16[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const uint32_t r = min(R * p + rr, a.vocab - 1);
            const uint32_t blk = r * 8 + b;
            const uint32_t lo = blk * 128 + 64 * hh + 32 * (k & 1), ho = blk * 64 + 32 * hh;
            l0[rr] = gnt4(hql, lo); l1[rr] = gnt4(hql, lo + 16); h0[rr] = gnt4(hqh, ho); h1[rr] = gnt4(hqh, ho + 16);
            const uint32_t so = blk * 16 + 8 * hh + 2 * k;
            s0[rr] = (int8_t)hsc[so]; s1[rr] = (int8_t)hsc[so + 1];
            d16[rr] = ld_u16(hd, blk * 2);
        }
        float part[R], out[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) part[rr] = dot_q6(l0[rr], l1[rr], h0[rr], h1[rr], s0[rr], s1[rr], d16[rr], ib, g, bias);
        rows_reduce<R>(part, out, lane);
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const uint32_t r = R * p + rr;
            if (r < a.vocab) {
                const float v = out[rr];
                if (!fin || !isfinite(v)) nf = true;
                if (lg && lane == rr) lg[r] = v;
                if (v > best) { best = v; besti = r; }   // rows ascend: ties keep the lower index
            }
        }
    }
    bv = best;
    bi = besti;
    nonfin = nf;
}

// total order of the argmax: larger value, then lower index (NaN below every number)
DEV bool better(float v, uint32_t i, float bv, uint32_t bi) { return v > bv || (v == bv && i < bi); }

}  // namespace

// ================================================================= kernel
extern "C" __global__ __launch_bounds__(NT, 1) void qxk_decode(QxDArgs args) {
    __shared__ DLds S;
    // the arguments are read from an LDS copy where used (LDS reads are not hoisted across
    // the stage barriers, so the ~70 argument dwords are not all held in scalar registers)
    __shared__ QxDArgs a;
    static_assert(sizeof(QxDArgs) % 8 == 0 && sizeof(QxDArgs) <= NT * 8, "argument copy");
    if (threadIdx.x < sizeof(QxDArgs) / 8)
        reinterpret_cast<uint64_t *>(&a)[threadIdx.x] = reinterpret_cast<const uint64_t *>(&args)[threadIdx.x];
    __syncthreads();
    const int wg = blockIdx.x;
    const Ctl ctl{gpw(a.abort), a.timeout};
    const uint32_t L = a.layers, E = a.experts;
    const uint32_t phases = QXD_PHASES(L);   // per step: 5 per layer, head input, argmax
    {
        const int tid = tix();
        for (int i = tid; i < 512; i += NT) S.g2[i] = a.T.g2[i];
        if (tid < 256) S.g3[tid] = a.T.g3[tid];
        if (tid < 128) S.sel[tid] = a.T.sel[tid];
    }
    WQ wq;
    WO wo;
    WE we;
    WD wd;
    AttnPre ap;
    float4 wm0 = make_float4(0.f, 0.f, 0.f, 0.f), wm1 = wm0;
    float fnw[8];
    load_wq(a, 0, wq);
    load_wo(a, 0, wo);
    uint32_t token = 0;
    __syncthreads();
    GLB uint64_t *const X = gpw(a.xch);
    for (uint32_t step = 0; step < a.steps; ++step) {
        const uint32_t pos = a.pos0 + step;
        const uint32_t ep_step = a.ep0 + step * phases + 1;
        const bool head_step = a.force_head || step + 1 >= a.n_prompt;
        const bool last = step + 1 == a.steps;
        if (step < a.n_prompt) token = gp(a.tokens)[step];
        // embedding row of the token (reference src/qx_format.c:3759-3793), decoded by every
        // workgroup into its copy of x
        if (tix() < 256) embed_q4k_row((const uint8_t *)(gp(a.emb) + (uint64_t)token * a.emb_row), S.xs);
        __syncthreads();
        for (uint32_t l = 0; l < L; ++l) {
            const uint32_t ep = ep_step + 5 * l;   // + 0 X, + 1 QKV, + 2 CX, + 3 XP/LG, + 4 H/WT
            const uint32_t par = l & 1;
            const uint32_t ln = l + 1 < L ? l + 1 : 0u;   // after the last layer: layer 0 of the next step
            // ---------------------------------------------------------- stage Q
            double a_part = 0.0;   // router x-part of expert wg (workgroups < E)
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                DMARK(l, 0);
                if (l > 0 && !wait_xch<4>(X + XO_X + par * XN_X, 2048, ep, reinterpret_cast<uint32_t *>(S.xs), Ident(), NWG,
                                          [](int j) { return 8 * j; }, S, ctl))
                    return;
                DMARK(l, 1);
                // the normalised input's digits; the attn-norm weights came with the Q/K/V rows
                double inv = 1.0;
                bool fin = true;
                {
                    double ss = 0.0;
                    if (tid < 256) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) ss += (double)S.xs[8 * tid + i] * (double)S.xs[8 * tid + i];
                    }
                    ss = wave_total_d(ss);
                    if (lane == 0) S.red[wave] = ss;
                    // router x-part: sum_i W[e,i] w_i x_i over values 4 tid .. 4 tid + 3
                    if ((uint32_t)wg < E) {
                        const float4 x4 = reinterpret_cast<const float4 *>(S.xs)[tid];
                        a_part = (double)wo.wr.x * (double)wo.fw.x * (double)x4.x + (double)wo.wr.y * (double)wo.fw.y * (double)x4.y +
                                 (double)wo.wr.z * (double)wo.fw.z * (double)x4.z + (double)wo.wr.w * (double)wo.fw.w * (double)x4.w;
                    }
                    __syncthreads();
                    const double tot = (S.red[0] + S.red[1]) + (S.red[2] + S.red[3]);
                    inv = 1.0 / sqrt(tot / 2048.0 + 1.0e-6);
                }
                if (tid < 256) {
                    float y[8];
                    const float nw8[8] = {wq.nw0.x, wq.nw0.y, wq.nw0.z, wq.nw0.w, wq.nw1.x, wq.nw1.y, wq.nw1.z, wq.nw1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) y[i] = (float)((double)S.xs[8 * tid + i] * inv) * nw8[i];
                    float mx = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) { fin = fin && isfinite(y[i]); mx = fmaxf(mx, fabsf(y[i])); }
                    mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
                    mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
                    uint32_t h0, h1, m0, m1, l0, l1;
                    float sc;
                    digits8(y, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
                    uint32_t *d = S.dig + (tid >> 2) * DIG_STRIDE;
                    const int q = tid & 3;
                    *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
                    *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
                    *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
                    if (q == 0) d[24] = __float_as_uint(sc);
                }
                if ((uint32_t)wg < E) {
                    a_part = wave_total_d(a_part);
                    if (lane == 0) S.red[NWV + wave] = a_part;
                }
                const bool ok = !block_any(!fin, S);
                DMARK(l, 13);
                if ((uint32_t)wg < E)
                    a_part = ((S.red[NWV + 0] + S.red[NWV + 1]) + (S.red[NWV + 2] + S.red[NWV + 3])) +
                             ((S.red[NWV + 4] + S.red[NWV + 5]) + (S.red[NWV + 6] + S.red[NWV + 7]));
                Dig g;
                load_dig(S.dig, lane, g);
                float part[4], out[4];
                part[0] = dot_iq4(wq.q[0], wq.m[0], ib, g);
                part[1] = dot_iq4(wq.q[1], wq.m[1], ib, g);
                part[2] = wave < 4 ? dot_iq4(wq.q[2], wq.m[2], ib, g) : 0.0f;
                part[3] = 0.0f;
                rows_reduce<4>(part, out, lane);
                // gather the workgroup's 20 rows, then one store: Q rows 16 wg .., K/V rows 4096 + 4 wg ..
#pragma unroll
                for (int r = 0; r < 3; ++r)
                    if (lane == r && (r < 2 || wave < 4)) {
                        const float v = (ok && isfinite(out[r])) ? out[r] : 0.0f;
                        S.outw[r < 2 ? 2 * wave + r : 16 + wave] = v;
                    }
                __syncthreads();
                if (tid < 20) {
                    GLB uint64_t *qkv = X + XO_QKV + par * XN_QKV;
                    xstf(qkv + (tid < 16 ? 16 * wg + tid : 4096 + 4 * wg + (tid - 16)), ep + 1, S.outw[tid]);
                }
                DMARK(l, 2);
            }
            // prefetch: the router fold rows (stage O); attention workgroups the cached K/V
            // rows they attend to, the others the next layer's Q/K/V rows
            load_wm(a, l, wm0, wm1);
            if (wg < QXG_HEADS) attn_prefetch(a, l, pos, ap);
            else load_wq(a, ln, wq);
            // ---------------------------------------------------------- stage A
            if (wg < QXG_HEADS) {
                if (!attn_wait(a, l, ep + 1, S, ctl)) return;
                DMARK(l, 3);
                attention(a, l, pos, ep + 1, ap, S);
                DMARK(l, 4);
            }
            // ---------------------------------------------------------- stage O
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                // sentinels: words 128 h and 128 h + 64 (the two store instructions of head h)
                if (!wait_xch<8>(X + XO_CX + par * XN_CX, 4096, ep + 2, S.u.vin, Ident(), 2 * QXG_HEADS,
                                 [](int j) { return 64 * j; }, S, ctl))
                    return;
                DMARK(l, 5);
                load_w8(plane(a, PL_FFN_NORM, l), fnw);   // for stage G
                if (wg < QXG_HEADS) load_wq(a, ln, wq);
                const float *cx = reinterpret_cast<const float *>(S.u.vin);
                double b_part = 0.0;
                if ((uint32_t)wg < E) {   // router ctx-part: sum_j M[e,j] ctx_j over values 8 tid ..
                    const float4 c0 = reinterpret_cast<const float4 *>(cx)[2 * tid], c1 = reinterpret_cast<const float4 *>(cx)[2 * tid + 1];
                    b_part = (double)wm0.x * (double)c0.x + (double)wm0.y * (double)c0.y + (double)wm0.z * (double)c0.z +
                             (double)wm0.w * (double)c0.w + (double)wm1.x * (double)c1.x + (double)wm1.y * (double)c1.y +
                             (double)wm1.z * (double)c1.z + (double)wm1.w * (double)c1.w;
                    b_part = wave_total_d(b_part);
                    if (lane == 0) S.red[wave] = b_part;
                    __syncthreads();   // (uniform: wg < E)
                    if (tid < 2) {   // the logit before the 1/rms(x') factor, (hi, lo) words
                        const double bsum = ((S.red[0] + S.red[1]) + (S.red[2] + S.red[3])) + ((S.red[4] + S.red[5]) + (S.red[6] + S.red[7]));
                        const uint64_t bits = (uint64_t)__double_as_longlong(a_part + bsum);
                        xst(X + XO_LG + par * XN_LG + 2 * wg + tid, ep + 3, tid == 0 ? (uint32_t)(bits >> 32) : (uint32_t)bits);
                    }
                }
                const bool ok = vec_digits<4096, false>(cx, nullptr, S);   // ends with barriers
                DMARK(l, 14);
                Dig g0, g1;
                load_dig(S.dig, lane, g0);
                load_dig(S.dig, lane + 64, g1);
                float part[1], out[1];
                part[0] = dot_iq4(wo.q0, wo.m0, ib, g0) + dot_iq4(wo.q1, wo.m1, ib, g1);
                rows_reduce<1>(part, out, lane);
                const int r = 8 * wg + wave;
                const float o = (ok && isfinite(out[0])) ? out[0] : 0.0f;
                if (lane == 0) S.outw[wave] = S.xs[r] + o;
                __syncthreads();
                if (tid < 8) xstf(X + XO_XP + par * XN_XP + 8 * wg + tid, ep + 3, S.outw[tid]);
                DMARK(l, 6);
            }
            // ---------------------------------------------------------- stage G
            uint32_t ids[QXG_TOPK];
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                const int gw = NWV * wg + wave;
                // the E router logits first (hi and lo words; sentinels: the hi words): the
                // top-8 and the routed experts' row loads then overlap the wait for x'
                if (!wait_xch<1, true>(X + XO_LG + par * XN_LG, 2 * (int)E, ep + 3, S.lgw, Ident(), (int)E,
                                 [](int j) { return 2 * j; }, S, ctl))
                    return;
                DMARK(l, 7);
                const uint32_t *lgw = S.lgw;
                auto logit = [&](uint32_t e) {
                    return __longlong_as_double((long long)(((uint64_t)lgw[2 * e] << 32) | lgw[2 * e + 1]));
                };
                // x' words read now, ahead of the expert rows in the load queue (they were
                // published before the router logits, so they are normally all there)
                const GLB uint64_t *xpb = X + XO_XP + par * XN_XP;
                uint64_t xpw[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) xpw[k] = xld(xpb + tid + NT * k);
                {   // every wave picks on its own (no barrier); ids are wave-uniform
                    const double l0 = lane < (int)E ? logit(lane) : 0.0, l1 = lane + 64 < (int)E ? logit(lane + 64) : 0.0;
                    wave_top8_ids(l0, l1, (int)E, ids);
#pragma unroll
                    for (int q = 0; q < QXG_TOPK; ++q) ids[q] = ids[q] < E ? ids[q] : 0u;
                }
                DMARK(l, 16);
                load_we(a, l, ids, we);
                load_wd(a, l, ids, wd);
                DMARK(l, 8);
                bool have = true;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    have = have && (uint32_t)(xpw[k] >> 32) == ep + 3;
                    reinterpret_cast<uint32_t *>(S.xp)[tid + NT * k] = (uint32_t)xpw[k];
                }
                if (block_any(!have, S) &&
                    !wait_xch<4>(xpb, 2048, ep + 3, reinterpret_cast<uint32_t *>(S.xp), Ident(), NWG, [](int j) { return 8 * j; }, S, ctl))
                    return;
                DMARK(l, 9);
                double inv = 1.0;
                (void)vec_digits<2048, true>(S.xp, fnw, S, &inv);   // h of a non-finite row is 0 by itself
                DMARK(l, 17);
                if (wg == 0 && wave == 0) {   // renormalised weights of the picks (reference :5265-5290)
                    const double l0 = lane < (int)E ? logit(lane) : 0.0, l1 = lane + 64 < (int)E ? logit(lane + 64) : 0.0;
                    double wts[QXG_TOPK];
                    wave_top8_weights(l0 * inv, l1 * inv, ids, wts);
                    if (lane < 2 * QXG_TOPK) {   // lane 2q: hi word of weight q, lane 2q + 1: lo word
                        double wl = 0.0;
                        uint32_t il = 0u;
#pragma unroll
                        for (int q = 0; q < QXG_TOPK; ++q) if ((lane >> 1) == q) { wl = wts[q]; il = ids[q]; }
                        const uint64_t bits = (uint64_t)__double_as_longlong(wl);
                        xst(X + XO_WT + par * XN_WT + lane, ep + 4, (lane & 1) ? (uint32_t)bits : (uint32_t)(bits >> 32));
                        if (last && a.d_rids && !(lane & 1)) { gpw(a.d_rids)[8 * l + (lane >> 1)] = il; gpw(a.d_rw)[8 * l + (lane >> 1)] = wl; }
                    }
                }
                Dig g;
                load_dig(S.dig, lane, g);
                float p[8], o[8];
#pragma unroll
                for (int uu = 0; uu < 3; ++uu) {
                    p[uu] = dot_iq2(we.gq[uu], we.gs[uu], we.gd[uu], g, S.g2, S.sel);
                    p[4 + uu] = dot_iq2(we.uq[uu], we.us[uu], we.ud[uu], g, S.g2, S.sel);
                }
                p[3] = p[7] = 0.0f;
                rows_reduce<8>(p, o, lane);
                DMARK(l, 18);
                (void)ib;
                (void)gw;
#pragma unroll
                for (int k = 0; k < 3; ++k)
                    if (lane == k) {
                        const float gv = isfinite(o[k]) ? o[k] : 0.0f, uv = isfinite(o[4 + k]) ? o[4 + k] : 0.0f;
                        // reference src/qx_format.c:5298, 2511-2513: h = (float)(silu((double)g) * (double)u)
                        const double sg = (double)gv / (1.0 + exp(-(double)gv));
                        S.outw[3 * wave + k] = (float)(sg * (double)uv);
                    }
                __syncthreads();
                if (tid < 24) xstf(X + XO_H + par * XN_H + 24 * wg + tid, ep + 4, S.outw[tid]);
                DMARK(l, 10);
            }
            // ---------------------------------------------------------- stage D
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6;
                // h (sentinels: word 24 g) and the 8 expert weights (hi, lo words; sentinel word 0)
                if (!wait_xch<13>(X, 6144 + 16, ep + 4, S.u.vin,
                                  [par](int i) { return i < 6144 ? (int)(XO_H + par * XN_H) + i : (int)(XO_WT + par * XN_WT) + i - 6144; },
                                  NWG + 1, [par](int j) { return j < NWG ? (int)(XO_H + par * XN_H) + 24 * j : (int)(XO_WT + par * XN_WT); },
                                  S, ctl))
                    return;
                DMARK(l, 11);
                load_wo(a, ln, wo);   // the next layer's O rows and router rows
                const uint32_t *wtw = S.u.vin + 6144;
                double wr[QXG_TOPK];
#pragma unroll
                for (int q = 0; q < QXG_TOPK; ++q)
                    wr[q] = __longlong_as_double((long long)(((uint64_t)wtw[2 * q] << 32) | wtw[2 * q + 1]));
                const bool okh = vec_digits<6144, false>(reinterpret_cast<const float *>(S.u.vin), nullptr, S);
                DMARK(l, 15);
                const int rk = lane >> 3, k = lane & 7;
                float part = 0.0f;
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    Dig g;
                    load_dig(S.dig, 24 * rk + 8 * j + k, g);
                    part += dot_iq3(wd.dq[j], wd.dax[j], wd.dd[j], g, S.g3, S.sel);
                }
                part += dppf<DPP_XOR1>(part);
                part += dppf<DPP_XOR2>(part);
                part += dppf<DPP_HALF_MIRROR>(part);   // lanes 8q..8q+7 hold rank q's row
                const float y = (okh && isfinite(part)) ? part : 0.0f;
                // reference src/qx_format.c:5296-5309: moe += (float)(w_r * (double)y_r), rank order
                float moe = 0.0f;
#pragma unroll
                for (int q = 0; q < QXG_TOPK; ++q) moe += (float)(wr[q] * (double)rdlanef(y, 8 * q));
                const int r = 8 * wg + wave;
                const float xn = S.xp[r] + moe;
                if (lane == 0) {
                    S.outw[wave] = xn;
                    if (last && a.d_layer) gpw(a.d_layer)[l * 2048 + r] = xn;
                    if (last && a.d_res && l + 1 == L) gpw(a.d_res)[r] = xn;
                }
                __syncthreads();
                if (tid < 8) xstf(X + XO_X + ((l + 1) & 1) * XN_X + 8 * wg + tid, ep + 5, S.outw[tid]);
                DMARK(l, 12);
            }
        }
        // ---------------------------------------------------------------- head
        if (head_step) {
            const int tid = tix(), lane = tid & 63, wave = tid >> 6;
            const uint32_t eph = ep_step + 5 * L;
            float onw[8];
            if (tid < 256) {
                const float4 x0 = ldf4((const GLB uint8_t *)gp(a.out_norm), 32 * tid), x1 = ldf4((const GLB uint8_t *)gp(a.out_norm), 32 * tid + 16);
                onw[0] = x0.x; onw[1] = x0.y; onw[2] = x0.z; onw[3] = x0.w; onw[4] = x1.x; onw[5] = x1.y; onw[6] = x1.z; onw[7] = x1.w;
            }
            DMARK(48, 0);
            if (!wait_xch<4>(X + XO_X + (L & 1) * XN_X, 2048, eph, reinterpret_cast<uint32_t *>(S.xs), Ident(), NWG,
                             [](int j) { return 8 * j; }, S, ctl))
                return;
            DMARK(48, 1);
            const bool fin = vec_digits<2048, true>(S.xs, onw, S);
            float bv;
            uint32_t bi;
            bool nonfin;
            DMARK(48, 2);
            head_rows<4>(a, S, fin, bv, bi, nonfin);
            DMARK(48, 3);
            // layer 0's rows again (also on the last step): they are then dead during the head
            // rows, whose loads take their registers
            load_wq(a, 0, wq);
            load_wo(a, 0, wo);
            if (nonfin) gpw(a.st)->nonfinite = 1u;
            // workgroup best, then every workgroup reads all the bests
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const uint32_t oi = __shfl_xor(bi, o);
                if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            if (lane == 0) { S.u.hd.bv[wave] = bv; S.u.hd.bi[wave] = bi; }
            __syncthreads();
            if (tid < 2) {
                float v = S.u.hd.bv[0];
                uint32_t i = S.u.hd.bi[0];
                for (int w = 1; w < NWV; ++w)
                    if (better(S.u.hd.bv[w], S.u.hd.bi[w], v, i)) { v = S.u.hd.bv[w]; i = S.u.hd.bi[w]; }
                xst(X + XO_AM + (step & 1) * XN_AM + 2 * wg + tid, eph + 1, tid == 0 ? __float_as_uint(v) : i);
            }
            if (!wait_xch<1>(X + XO_AM + (step & 1) * XN_AM, XN_AM, eph + 1, S.u.hd.am, Ident(), NWG,
                             [](int j) { return 2 * j; }, S, ctl))
                return;
            DMARK(48, 4);
            float v = __uint_as_float(S.u.hd.am[0]);
            uint32_t i = S.u.hd.am[1];
            for (int w = 1; w < NWG; ++w) {
                const float ov = __uint_as_float(S.u.hd.am[2 * w]);
                const uint32_t oi = S.u.hd.am[2 * w + 1];
                if (better(ov, oi, v, i)) { v = ov; i = oi; }
            }
            token = i < a.vocab ? i : 0u;
            if (wg == 0 && tid == 0 && step + 1 >= a.n_prompt) gpw(a.tokens)[step + 1] = token;
            __syncthreads();
        }
    }
}

// Router fold of one layer (see the top of this file): M[e][j] = sum_i W[e][i] w[i] O[i][j]
// in double, stored as f32, with O [2048][4096] the layer's dequantized O projection
// (bit-exact, qxk_dequant) and w the ffn-norm weights.  Grid (16, ceil(E / 4)) of 256
// threads: thread j of 4 experts.
extern "C" __global__ __launch_bounds__(256) void qxk_router_fold(const float *W, const float *w, const float *O,
                                                                   uint32_t E, float *M) {
    __shared__ double sw[4][2048];
    const uint32_t e0 = blockIdx.y * 4, j = blockIdx.x * 256 + threadIdx.x;
    for (int i = threadIdx.x; i < 2048; i += 256)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            sw[k][i] = e0 + k < E ? (double)W[(uint64_t)(e0 + k) * 2048 + i] * (double)w[i] : 0.0;
    __syncthreads();
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int i = 0; i < 2048; ++i) {
        const double o = (double)O[(uint64_t)i * 4096 + j];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = fma(sw[k][i], o, acc[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (e0 + k < E) M[(uint64_t)(e0 + k) * 4096 + j] = (float)acc[k];
}
