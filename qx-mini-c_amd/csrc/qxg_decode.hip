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

// Stage timestamps for development builds only (-DQXD_TRACE): on the last step, one lane
// per workgroup records s_memrealtime (100 MHz) for layers 20..23 and the head into LDS
// (a global store would count in the wave's vmcnt and delay the next poll); after the step
// loop the workgroup copies them to qxd_trace_buf[layer][point][workgroup], read back with
// qxd_trace_read.
#ifdef QXD_TRACE
__device__ unsigned long long qxd_trace_buf[49][40][256];
__shared__ unsigned long long qxd_tl[5][40];
extern "C" int qxd_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(qxd_trace_buf), sizeof(qxd_trace_buf)) == hipSuccess;
}
#define QXD_TL_SLOT(layer) ((layer) >= 20 && (layer) < 24 ? (int)(layer) - 20 : (layer) == 48 ? 4 : -1)
#define DMARKT(layer, point, thread)                                                                           \
    do {                                                                                                      \
        const int sl_ = QXD_TL_SLOT(layer);                                                                   \
        if (last && sl_ >= 0 && (threadIdx.x == (thread))) qxd_tl[sl_][point] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define DMARK(layer, point) DMARKT(layer, point, 0)
#else
#define DMARK(layer, point) ((void)0)
#define DMARKT(layer, point, thread) ((void)0)
#endif

// First-round delays of five exchange polls (x in stage Q, x' in stage G, h in stage D, the
// chunk records of the chunked stage A's merge and, in the chunked kernel, the context in
// stage O), in units of 64 cycles (s_sleep).  A workgroup reaches a poll right after storing its own
// outputs, ahead of most producers, and poll rounds issued while the words are still in
// flight only load the memory system that the producers' stores and the weight copies go
// through.  Measured on the benchmark: 24 (~0.64 us) for x and the merge, 16 (~0.43 us) for
// x', h and the chunked kernel's context (every workgroup publishes 16 merged dimensions,
// then polls all 4096); longer or shorter was slower, a sleep between rounds was slower, and
// delaying the other polls (the walk kernel's context among them) gave nothing.
#ifndef QXD_SLEEP_X
#define QXD_SLEEP_X 24
#endif
#ifndef QXD_SLEEP_XP
#define QXD_SLEEP_XP 16
#endif
#ifndef QXD_SLEEP_H
#define QXD_SLEEP_H 16
#endif
#ifndef QXD_SLEEP_MG
#define QXD_SLEEP_MG 24
#endif
#ifndef QXD_SLEEP_CX
#define QXD_SLEEP_CX 16
#endif
#define QXD_SLEEP(n) \
    do { \
        if ((n) > 0) __builtin_amdgcn_s_sleep((n) > 0 ? (n) : 1); \
    } while (0)

namespace {

constexpr int NT = 512;            // threads per workgroup
constexpr int NWV = NT / 64;       // waves per workgroup
constexpr int NWG = QXG_PBLOCKS;   // workgroups, one per CU
static_assert((NWG - QXG_HEADS) * 24 >= 5120, "the non-attention workgroups' 24 slots cover the Q/K/V rows");
constexpr uint32_t GU_BYTES = 4096, DN_BYTES = 3072;   // per-wave LDS for the routed experts' rows
constexpr int HEAD_R = 4;                                // head rows per wave and pass
constexpr int HEAD_NI = (HEAD_R * 105 + 63) / 64;        // 16-byte load instructions per pass
#ifndef QXD_TLB_PAGE
#define QXD_TLB_PAGE (2ull << 20)
#endif

// exchange buffers: word offsets of slot 0 (slot 1 follows at + size)
constexpr uint32_t XN_X = 2048, XN_QKV = 5120, XN_CX = 4096, XN_XP = 2048, XN_LG = 256, XN_H = 6144, XN_WT = 16,
                   XN_AM = 2 * NWG, XN_PT = QXD_PART_WORDS;   // (partial results: their own buffer)
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
DEV void xst(GLB uint64_t *p, uint32_t ep, uint32_t bits) {
    __hip_atomic_store(p, ((uint64_t)ep << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void xstf(GLB uint64_t *p, uint32_t ep, float v) { xst(p, ep, __float_as_uint(v)); }
DEV void st_coherent(GLB uint32_t *p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

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
struct AttnW {                   // one wave's attention scratch
    int8_t kc[128], vc[128];     // the position's K and V codes of the workgroup's kv head
    float p[16];                 // weights of the wave's positions in the current block
};
struct AttnS {
    float q[128], k[512], v[512];   // polled q of the head, K and V rows (all four kv heads)
    uint32_t qd[4 * DIG_STRIDE];    // q digit planes
    float kmx[4], vmx[4];           // largest magnitudes of the K and V rows per kv head
    uint32_t qok;
    AttnW w[NWV];
    int8_t kq[512], vq[512];        // the position's INT8 K and V rows (cache store)
    float ctx[NWV][128];            // per wave: context partial sums
    double m[NWV], l[NWV];          // per wave: running maximum and denominator
};
struct AttnK {                      // stage A by kv head and position chunk (attention_chunk_part)
    float q[NWV][128];              // polled q of heads 8 g .. 8 g + 7, normalised and rotated in place
    float k[512], v[512];           // the position's K and V rows (all four kv heads); follow q for the poll
    uint32_t qd[NWV][4 * DIG_STRIDE];   // each head's q digit planes
    float kmx[4], vmx[4];           // largest magnitudes of the K and V rows per kv head
    uint32_t qok[NWV];
    float p[NWV][QXD_CHUNK];        // per wave: weights of the chunk's positions (0 past the position)
};
struct ChunkRows {                  // the chunk's cached K and V rows of kv head g and their scales,
    alignas(16) int8_t k[QXD_CHUNK][128];   // copied to LDS in stage Q (dma_chunk); rows past the
    alignas(16) int8_t v[QXD_CHUNK][128];   // position repeat its predecessor's and are masked
    float ks[QXD_CHUNK], vs[QXD_CHUNK];
};
struct DLds {
    uint4 g2[512];
    uint2 g3[256];
    uint2 sel[128];
    float xs[2048];              // layer input x (stage Q .. O residual)
    float xp[2048];              // x' = x + O ctx (stage G .. D residual)
    uint32_t dig[192 * DIG_STRIDE];
    uint4 wq[NWV][3][64];        // Q/K/V qs chunks of each wave (DMA, one layer ahead)
    uint4 wo[NWV][2][64];        // O qs chunks of each wave (DMA, one layer ahead)
    double red[2 * NWV];
    uint32_t lgw[2 * 128];       // router logits (hi, lo words)
    double xinv;                 // 1 / rms(x') (stage G)
    float ys[QXG_TOPK][8];       // down rows of each rank (stage D)
    float outw[32];              // the workgroup's outputs of a stage, gathered for one store
    float oatt[NWV];             // the workgroup's O-projection outputs (stage O, for the last step's dumps)
    uint32_t flag[NWV];
    uint32_t bflag[2][NWV];      // block_any flags, two sets by call parity
    uint32_t bpar[NWV];          // block_any call parity of each wave
    uint32_t sub[4];             // upper_waves_sync flags of waves 4..7
    uint32_t sublo[4];           // lower_waves_sync flags of waves 0..3
    uint32_t fail;               // a poll of waves 4..7 timed out (stage G)
    double ssp[4];               // x' sums of squares of waves 4..7 (stage G)
    uint32_t dne[QXG_TOPK];      // the picked experts by rank (stage G, for stage D's down rows)
    union {
        struct {
            union {
                alignas(16) uint32_t vin[6144 + 16];    // polled ctx (4096), or h (6144) and the 8 expert weights
                alignas(16) uint8_t gu[NWV][GU_BYTES];  // gate/up rows of each wave (DMA and dots in stage G)
            };
            alignas(16) uint8_t dn[NWV][DN_BYTES];      // down rows of each wave (DMA in stage G, dots in stage D)
        } m;
        AttnS att;
        AttnK atk;
        struct {
            float bv[NWV];
            uint32_t bi[NWV];
            uint32_t next;           // the head's group counter (head_rows)
            uint32_t am[XN_AM];
            alignas(16) uint8_t rows[NWV][HEAD_NI * 1024];   // each wave's staged head rows
        } hd;
    } u;
};

// block-wide OR of a per-thread flag (every thread of the workgroup calls it); includes
// the barrier that publishes the caller's earlier LDS writes.  One barrier: the flags
// alternate between two sets by call parity (each wave keeps its own parity bit), and a
// wave can only write a set again two calls later, after the barrier of the call between,
// which every wave reaches after reading this call's set.
DEV bool block_any(bool f, DLds &S) {
    const bool any = __ballot(f) != 0;
    const int wave = threadIdx.x >> 6;
    const uint32_t p = S.bpar[wave];   // (only this wave touches its bit)
    if ((threadIdx.x & 63) == 0) {
        S.bflag[p][wave] = any ? 1u : 0u;
        S.bpar[wave] = p ^ 1u;
    }
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) r |= S.bflag[p][w];
    return r != 0;
}

// A workgroup's wait for an exchange, by direct polling: thread t reads word pairs
// (2 p, 2 p + 1), p = t + 512 k, with one 16-byte agent-scope load each (two tagged words;
// each 8-byte half is read whole, as a 64-bit load would), and re-reads only the pairs not
// yet carrying epoch ep.  One round trip once the words are there; measured on the GPU,
// an all-to-all of 6144 words completes in 2.7 us this way against 4.5 us with a sentinel
// phase and 64-bit loads (the vector-memory unit takes about the same time per load
// instruction whatever its width).  idx(i) maps word i < n (n even) to its offset from
// base; pairs are contiguous (idx(2p + 1) = idx(2p) + 1) and 16-byte aligned.  All threads
// call it; the payloads are in dst (LDS) when it returns true.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
DEV void ld_pair(u32x4 &v, const GLB uint64_t *p) {
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
}
template <int K2>
DEV void wait_pairs(u32x4 (&w)[K2]) {
    static_assert(K2 >= 1 && K2 <= 7, "pairs per thread");
    if constexpr (K2 == 1) asm volatile("s_waitcnt vmcnt(0)" : "+v"(w[0]) : : "memory");
    else if constexpr (K2 == 2) asm volatile("s_waitcnt vmcnt(0)" : "+v"(w[0]), "+v"(w[1]) : : "memory");
    else if constexpr (K2 == 4) asm volatile("s_waitcnt vmcnt(0)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]) : : "memory");
    else if constexpr (K2 == 7)
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]) : : "memory");
    else static_assert(K2 == 1 || K2 == 2 || K2 == 4 || K2 == 7, "pairs per thread");
}
// The polling of wait_xch2 by threads T0 .. T0 + P - 1 only (the caller's branch), pair
// p = t + P k for thread T0 + t; returns this thread's success, with no barrier.  ssq (may
// be null) gets the sum of squares of the thread's payloads as f32 values, in double.
template <int K2, int P = NT, int T0 = 0, typename IDX>
DEV bool poll_pairs(const GLB uint64_t *base, int n, uint32_t ep, uint32_t *dst, IDX idx, const Ctl &c,
                    double *ssq = nullptr) {
    const int tid = tix() - T0;
    u32x4 w[K2];
    bool got[K2];
#pragma unroll
    for (int k = 0; k < K2; ++k) {
        const int i = 2 * (tid + P * k);
        got[k] = i >= n;
        w[k] = u32x4{0u, ep, 0u, ep};
    }
    const uint64_t deadline = wall_clock64() + c.timeout;
    uint32_t it = 0;
    bool ok = true;
    for (;;) {
#pragma unroll
        for (int k = 0; k < K2; ++k)
            if (!got[k]) ld_pair(w[k], base + idx(2 * (tid + P * k)));
        wait_pairs<K2>(w);
        bool all = true;
#pragma unroll
        for (int k = 0; k < K2; ++k) {
            got[k] = got[k] || (w[k].y == ep && w[k].w == ep);
            all = all && got[k];
        }
        if (all) break;
        if (!keep_waiting(it, deadline, c)) { ok = false; break; }
    }
#pragma unroll
    for (int k = 0; k < K2; ++k) {
        const int i = 2 * (tid + P * k);
        if (i < n) {
            *reinterpret_cast<uint2 *>(dst + i) = make_uint2(w[k].x, w[k].z);
            if (ssq) {
                const double u = (double)__uint_as_float(w[k].x), v = (double)__uint_as_float(w[k].z);
                *ssq += u * u + v * v;
            }
        }
    }
    return ok;
}
template <int K2, typename IDX>
DEV bool wait_xch2(const GLB uint64_t *base, int n, uint32_t ep, uint32_t *dst, IDX idx, DLds &S, const Ctl &c) {
    return !block_any(!poll_pairs<K2>(base, n, ep, dst, idx, c), S);
}

// Waves 4..7 only, all four calling it: each wave's earlier LDS writes are visible to the
// other three afterwards (the other four waves are not involved).  Each wave posts tag in its
// LDS flag, then spins on the four flags; tag must differ from every earlier call's (the
// exchange epochs are).  Every wave reaches its post, so the spin ends.
DEV void upper_waves_sync(DLds &S, uint32_t tag) {
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    const int wave = tix() >> 6;
    if ((tix() & 63) == 0) __hip_atomic_store(&S.sub[wave - 4], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (;;) {
        bool all = true;
#pragma unroll
        for (int w = 0; w < 4; ++w) all = all && __hip_atomic_load(&S.sub[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == tag;
        if (all) break;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
}

// The same for waves 0..3 (the other four not involved).
DEV void lower_waves_sync(DLds &S, uint32_t tag) {
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    const int wave = tix() >> 6;
    if ((tix() & 63) == 0) __hip_atomic_store(&S.sublo[wave], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (;;) {
        bool all = true;
#pragma unroll
        for (int w = 0; w < 4; ++w) all = all && __hip_atomic_load(&S.sublo[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == tag;
        if (all) break;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
}

// Chunk c (values 8 c .. 8 c + 7, in y) of a q8_k_compat activation into the digit planes:
// its Q8_K codes (q8_chunk: every lane of the wave calls it, 32 lanes a 256-value block) in
// the h plane, m = l = 0, and the block's d / 65536 as the 32-group scale, so the digit dots
// compute d * sum(code * w) (the per-phase kernels' block_q8).
DEV void store_q8(const float (&y)[8], int c, uint32_t *dig) {
    uint32_t h0, h1;
    const float dq = q8_chunk(y, h0, h1);
    uint32_t *d = dig + (c >> 2) * DIG_STRIDE;
    const int q = c & 3;
    *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
    *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(0u, 0u);
    *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(0u, 0u);
    if (q == 0) d[24] = __float_as_uint(dq * (1.0f / 65536.0f));
}

// Digit planes of an N-vector held in LDS (as f32 bits), 8 values per thread-chunk; with
// NORM it is first RMS-normalised (reference src/qx_format.c:3358-3371), w8 the norm
// weights of the thread's 8 values (threads < 256).
// The inverse RMS goes to *inv_out.  Returns true when every value is finite.  Q8: the
// q8_k_compat activations instead (Q8_K codes in the h plane, m = l = 0, each 32-group
// scale d / 65536; q8_chunk): the 256-value blocks are the chunks of 32 consecutive lanes.
template <int N, bool NORM, bool Q8 = false>
DEV bool vec_digits(const float *v, const float *w8, DLds &S, double *inv_out = nullptr, GLB float *norm_out = nullptr) {
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
            if (norm_out) {
#pragma unroll
                for (int i = 0; i < 8; ++i) norm_out[8 * c + i] = y[i];
            }
        }
        if constexpr (Q8) {   // (whole waves take each pass: NCH and NT are multiples of 64)
#pragma unroll
            for (int i = 0; i < 8; ++i) fin = fin && isfinite(y[i]);
            store_q8(y, c, S.dig);
        } else {
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
DEV uint2 gnt2(const GLB uint8_t *b, uint32_t off) {
    const u32x2 v = __builtin_nontemporal_load((const GLB u32x2 *)(b + off));
    return make_uint2(v.x, v.y);
}
DEV float4 ldf4(const GLB uint8_t *b, uint32_t off) {
    const f32x4 v = *(const GLB f32x4 *)(b + off);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Weight rows staged in LDS by the load-to-LDS path (global_load_lds_dwordx4): lane i's 16
// bytes land at lds + 16 i.  Issued as inline assembly so the compiler neither holds the
// rows in registers across the stages in between nor orders the workgroup's other LDS
// accesses behind the copy; the reader waits for it explicitly (wait_loads) at a point
// where no later-issued load is outstanding.  Non-temporal, as every weight byte.
DEV void dma16(const GLB uint8_t *base, uint32_t off, const void *lds) {
    const uint32_t l = (uint32_t)(uintptr_t)lds;   // low half of the flat address = LDS offset
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" : : "v"(off), "s"(base), "s"(l) : "memory", "m0");
}
// s_waitcnt vmcnt(0) as the builtin (0x0F70: vmcnt 0, expcnt and lgkmcnt unconstrained), which
// the compiler's wait insertion takes into account (after an opaque asm wait it still assumed
// older loads pending and waited again behind loads issued later); the fence keeps LDS reads
// of the copied rows below it.
DEV void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }
// The same copies with agent-coherent (sc1) loads, for KV-cache rows and scales, which
// workgroups of this launch store with agent-scope stores (every KV-cache read is
// agent-coherent): 16 bytes a lane, or 4 (lane i's at lds + 4 i).
DEV void dma16_kv(const GLB uint8_t *base, uint32_t off, const void *lds) {
    const uint32_t l = (uint32_t)(uintptr_t)lds;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc1" : : "v"(off), "s"(base), "s"(l) : "memory", "m0");
}
DEV void dma4_kv(const GLB uint8_t *base, uint32_t off, const void *lds) {
    const uint32_t l = (uint32_t)(uintptr_t)lds;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1 sc1" : : "v"(off), "s"(base), "s"(l) : "memory", "m0");
}

// layer l's plane `id` (scalar arithmetic on the argument copy)
DEV const GLB uint8_t *plane(const QxDArgs &a, int id, uint32_t l) {
    return (const GLB uint8_t *)(uni64((uint64_t)a.P[id].base) + (uint64_t)l * uni64(a.P[id].stride));
}
// decode pack w of layer l (the calling workgroup's by default)
DEV const GLB uint8_t *wg_pack(const QxDArgs &a, uint32_t l, uint32_t w = blockIdx.x) {
    return (const GLB uint8_t *)(uni64((uint64_t)a.PK.base) + (uint64_t)l * uni64(a.PK.stride) + (uint64_t)w * QXD_PK_BYTES);
}
// the pack holding the router and router-fold rows the workgroup reads: workgroups past the
// experts read expert E - 1's (unused) from one pack, so the copies stay in L2
DEV const GLB uint8_t *router_pack(const QxDArgs &a, uint32_t l) { return wg_pack(a, l, min((uint32_t)blockIdx.x, a.experts - 1u)); }

// ---------------------------------------------------------------- weight sets
// Q/K/V rows of a wave of workgroup wg >= QXG_HEADS (the attention workgroups make none):
// stacked rows [Q 4096 | K 512 | V 512] 24 (wg - 32) + 3 w + {0, 1, 2} (pack slots past row
// 5119 are zero), and the attn-norm weights of the thread's 8 values.
// The 16-byte qs chunks go to LDS (lq[wave][r][lane], DMA); meta and norm weights stay in
// registers.
struct WQ {
    uint2 m[3];
    float4 nw0, nw1;
};
DEV void load_wq(const QxDArgs &a, uint32_t l, WQ &w, uint4 (*lq)[64]) {
    const int tid = tix(), lane = tid & 63;
    const int wave = wave_id();
    const uint32_t b = lane >> 3, ib = lane & 7;
    const GLB uint8_t *pk = wg_pack(a, l);
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        const uint32_t blk = (uint32_t)(3 * wave + r) * 8 + b;
        dma16(pk, QXD_PK_QQ + blk * 128 + 16 * ib, lq[r]);
        w.m[r] = gnt2(pk, QXD_PK_QM + blk * 8);
    }
    const GLB uint8_t *nw = plane(a, PL_ATTN_NORM, l);
    w.nw0 = ldf4(nw, 32 * (tid & 255));
    w.nw1 = ldf4(nw, 32 * (tid & 255) + 16);
}
// O row 8 wg + w (16 blocks; lane takes blocks lane/8 and 8 + lane/8, sub-block lane%8)
// and router row W[e] with the ffn-norm weights, values 4 tid .. 4 tid + 3 (the router's
// x-part; workgroups e >= experts load an unused copy)
struct WO {
    uint2 m0, m1;
    float4 wr, fw;
};
// The O rows (load-to-LDS copies, which issue slowly: issued where the workgroup waits
// anyway, after its Q/K/V rows) ...
DEV void load_o(const QxDArgs &a, uint32_t l, WO &w, uint4 (*lo)[64]) {
    const int lane = tix() & 63;
    const int wave = wave_id();
    const uint32_t ib = lane & 7;
    const GLB uint8_t *pk = wg_pack(a, l);   // O rows 8 wg ..
    const uint32_t r = (uint32_t)wave * 16;
    const uint32_t k0 = r + (lane >> 3), k1 = r + 8 + (lane >> 3);
    dma16(pk, QXD_PK_OQ + k0 * 128 + 16 * ib, lo[0]);
    dma16(pk, QXD_PK_OQ + k1 * 128 + 16 * ib, lo[1]);
    w.m0 = gnt2(pk, QXD_PK_OM + k0 * 8);
    w.m1 = gnt2(pk, QXD_PK_OM + k1 * 8);
}
// ... and the router row min(wg, experts - 1) with the ffn-norm weights (register loads,
// needed from stage Q on)
DEV void load_wr(const QxDArgs &a, uint32_t l, WO &w) {
    const int tid = tix();
    w.wr = ldf4(router_pack(a, l), QXD_PK_RT + 16 * tid);
    w.fw = ldf4(plane(a, PL_FFN_NORM, l), 16 * tid);
}
// router fold row M[e], values 8 tid .. 8 tid + 7 (the router's ctx-part)
DEV void load_wm(const QxDArgs &a, uint32_t l, float4 &m0, float4 &m1) {
    const int tid = tix();
    const GLB uint8_t *pk = router_pack(a, l);
    m0 = ldf4(pk, QXD_PK_MF + 32 * tid);
    m1 = ldf4(pk, QXD_PK_MF + 32 * tid + 16);
}
// norm weights of the thread's 8 values 8 tid .. 8 tid + 7 (used by threads < 256; the
// others load a copy)
DEV void load_w8(const GLB uint8_t *p, float (&w)[8]) {
    const uint32_t t = tix() & 255;
    const float4 x0 = ldf4(p, 32 * t), x1 = ldf4(p, 32 * t + 16);
    w[0] = x0.x; w[1] = x0.y; w[2] = x0.z; w[3] = x0.w;
    w[4] = x1.x; w[5] = x1.y; w[6] = x1.z; w[7] = x1.w;
}
// Routed experts' rows, staged in LDS as whole 16-byte chunks (a CU's vector-memory unit
// spends about the same time per load instruction whatever its width).  A gate/up unit sits
// at uu * QXD_GU_UNIT: gate qs +0, sc +512, d +576, up qs +592, sc +1104, d +1168.
constexpr uint32_t GU_GSC = 512, GU_GD = 576, GU_UQ = 592, GU_USC = 1104, GU_UD = 1168;
// Gate/up dots of NU units at ub (LDS, QXD_GU_UNIT apart) for lane (b, ib) of each 32-value
// sub-block: p[k] gate and p[4 + k] up of unit k (the rest 0).  Sub-blocks in the order gate,
// up of unit 0, 1, ..; a sub-block's index words are read two ahead and its codebook entries
// one ahead of its dot.
template <int NU, bool H1 = false>
DEV void gu_dots(const uint8_t *ub, uint32_t q, uint32_t sc, uint32_t d, const DLds &S, const Dig &g, float (&p)[8]) {
    constexpr int NS = 2 * NU;
    uint2 qs[3];
    uint32_t scs[3], ds[3];
    auto ld = [&](int s2) {
        const uint8_t *u = ub + (s2 >> 1) * QXD_GU_UNIT;
        const bool up = s2 & 1;
        const uint32_t oq = up ? GU_UQ : 0u, os = up ? GU_USC : GU_GSC, od = up ? GU_UD : GU_GD;
        qs[s2 % 3] = *reinterpret_cast<const uint2 *>(u + oq + q);
        scs[s2 % 3] = u[os + sc];
        ds[s2 % 3] = *reinterpret_cast<const uint16_t *>(u + od + d);
    };
    ld(0);
    ld(1);
    Iq2Look kl[2];
    iq2_look(qs[0], S.g2, S.sel, kl[0]);
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) {
        if (s2 + 2 < NS) ld(s2 + 2);
        if (s2 + 1 < NS) iq2_look(qs[(s2 + 1) % 3], S.g2, S.sel, kl[(s2 + 1) & 1]);
        p[(s2 & 1) ? 4 + (s2 >> 1) : (s2 >> 1)] = iq2_dot<H1, true>(kl[s2 & 1], scs[s2 % 3], ds[s2 % 3], g);
    }
#pragma unroll
    for (int k = NU; k < 4; ++k) p[k] = p[4 + k] = 0.0f;
}
// The workgroup's 24 units (24 wg .. 24 wg + 23 of the stacked 8 x 768, one rank: 24 | 768)
// lie contiguously in HBM (28,416 bytes, 1776 chunks); wave w < 4 loads chunks 448 w ..
// 448 w + 447 (7 instructions, chunks past 1775 repeat the last one) to LDS byte 16 chunk.
DEV void addr_gu_wg(const uint32_t (&ids)[QXG_TOPK], int w, uint64_t gu_base, uint64_t (&addr)[7], uint32_t (&lds_off)[7]) {
    const int lane = tix() & 63;
    const uint32_t u0 = 24u * blockIdx.x, rank = u0 / QXG_FFN;
    uint32_t e = 0u;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q)
        if ((uint32_t)q == rank) e = ids[q];
    const uint64_t base = gu_base + (uint64_t)(e * QXG_FFN + u0 % QXG_FFN) * QXD_GU_UNIT;
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const uint32_t c = min(448u * w + 64u * i + lane, 24u * QXD_GU_UNIT / 16 - 1u);
        addr[i] = base + 16 * c;
        lds_off[i] = 16 * c;
    }
}
// Down rows 8 wg .. 8 wg + 7 of the expert of rank w: 8 * QXD_DN_ROW = 2432 contiguous bytes,
// chunks [0, 152) (3 instructions, 3 KB of LDS; lanes past 152 repeat chunk 0).  In LDS row
// j sits at j * QXD_DN_ROW: qs +0 (3 x 64), aux +192 (3 x 32), d +288 (3 x 2).  In HBM the
// 8-row blocks of all E experts for one row range lie together ((wg * E + e) * 8 rows), so a
// workgroup's 8 experts' down rows lie within E * 2432 bytes (311 KB at E = 128: one or two
// 2 MB translation pages instead of eight).
DEV void dma_dn(const QxDArgs &a, uint32_t l, uint32_t e, uint32_t E, uint8_t *lds) {
    const int lane = tix() & 63;
    const GLB uint8_t *base = (const GLB uint8_t *)uni64(uni64((uint64_t)a.DN.base) + (uint64_t)l * uni64(a.DN.stride) +
                                                          ((uint64_t)blockIdx.x * E + e) * (8 * QXD_DN_ROW));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const uint32_t c = 64 * i + lane;
        dma16(base, c < 8 * QXD_DN_ROW / 16 ? 16 * c : 0u, lds + 1024 * i);
    }
}
// The rows go through registers: 16-byte non-temporal loads, then one LDS store per chunk
// (the load-to-LDS path issues these copies far more slowly: measured 2.4 us for 14 per
// wave against 1.1 for 7).
template <int N>
DEV void load_rows(const uint64_t (&addr)[N], u32x4 (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = __builtin_nontemporal_load((const GLB u32x4 *)addr[i]);
}
template <int N>
DEV void store_rows(const u32x4 (&v)[N], uint8_t *lds) {
    const int lane = tix() & 63;
#pragma unroll
    for (int i = 0; i < N; ++i) *reinterpret_cast<u32x4 *>(lds + 1024 * i + 16 * lane) = v[i];
}

// ---------------------------------------------------------------- attention (stage A)
// Workgroup h: q head h (reference qx_rope_gqa_attention_partial, src/qx_format.c:5051-5196,
// and the state loop's K/V handling, 6282-6363): per-head q/k RMSNorm (3740-3757), RoPE
// (4625-4641, host table), INT8 K/V quantization of the position over all 512 values
// (4449-4463; workgroup 0 stores the rows, every workgroup derives the same row), scores of
// q as int8 digit planes against the INT8 K codes (v_dot4, exact), double softmax, f32
// context.
//
// Every wave works on its own until one barrier: it normalises and rotates the k of all four
// kv heads (the INT8 scale is over the whole 512-value row) and its q, forms the position's
// codes, then takes positions 128 i + 16 w .. + 15 (wave w, a quad per position) with an
// online softmax: running maximum m, denominator l and f32 context partial sums, rescaled
// by exp(m_old - m_new) when the maximum grows.  After the barrier thread d < 128 merges the
// eight waves: ctx[d] = sum_w (float)(exp(m_w - M) / L) * acc_w[d], L = sum_w exp(m_w - M) l_w
// (the same quantity as the reference's sum of exp(s - max) / den, within f32 roundings).
//
// The cached rows of positions 16 w + j (j < 16) are fetched before the Q/K/V exchange is
// polled (their addresses depend only on the layer and the position count): lane q of the
// quad of position 16 w + j takes the 32 K bytes of group q and the K and V scales, and lane
// (p, g) (p = lane / 16, g = lane % 16) the 8 V bytes of dims 8 g .. of positions 16 w + 4 i + p.
struct AttnPre {   // vector-typed fields: they stay in registers (arrays filled in branches did not)
    u32x4 k0, k1;
    float ks, vs;      // K and V scales of the quad's position
    u32x2 v0, v1, v2, v3;
    double cs, sn;     // RoPE table entries of the position, dims lane and lane + 64
    float nq0, nq1, nk0, nk1;   // q- and k-norm weights, dims lane, lane + 64
};
// KV cache reads: agent-coherent (sc1) buffer loads, 16/8/4 bytes per lane.  Rows written
// earlier in this launch were stored by workgroup 0 with agent-scope stores; every row is
// read the same way.  The base goes through readfirstlane: a descriptor the compiler cannot
// prove uniform (the argument copy is read from LDS) gets a loop around each load that
// copies the result out afterwards, which waits for the load right after issuing it.
constexpr int CP_SC1 = 16;
template <typename T>
DEV __amdgpu_buffer_rsrc_t rsrc(const T *p) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)uni64((uint64_t)p), (short)0, 0x7fffffff, 0x00020000);
}
DEV u32x4 kv_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP_SC1); }
DEV u32x2 kv_ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP_SC1); }
DEV uint32_t kv_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP_SC1); }

// the cached rows of one 128-position block (t0 = 128 i) for the calling lane, clamped to
// positions below pos (the position itself comes from the wave's own codes)
struct AttnRows {
    u32x4 k0, k1;
    float ks, vs;
    u32x2 v[4];
};
DEV void attn_rows(const QxDArgs &a, uint32_t l, uint32_t pos, uint32_t t0, AttnRows &r) {
    const int lane = tix() & 63, w = wave_id();
    const int kvh = blockIdx.x >> 3;
    const auto kr = rsrc(a.kc), vr = rsrc(a.vc), ksr = rsrc(a.ks), vsr = rsrc(a.vs);
    const uint32_t base = l * a.ctx, last = pos > 0 ? pos - 1 : 0u;
    const uint32_t tq = min(t0 + 16u * w + (lane >> 2), last);
    const uint32_t off = ((base + tq) * 128 + 32 * kvh + 8 * (lane & 3)) * 4;
    r.k0 = kv_ld16(kr, off);
    r.k1 = kv_ld16(kr, off + 16);
    r.ks = __uint_as_float(kv_ld4(ksr, (base + tq) * 4));
    r.vs = __uint_as_float(kv_ld4(vsr, (base + tq) * 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t tv = min(t0 + 16u * w + 4u * i + (lane >> 4), last);
        r.v[i] = kv_ld8(vr, ((base + tv) * 128 + 32 * kvh + 2 * (lane & 15)) * 4);
    }
}

DEV void attn_prefetch(const QxDArgs &a, uint32_t l, uint32_t pos, AttnPre &p) {
    AttnRows r;
    attn_rows(a, l, pos, 0u, r);
    p.k0 = r.k0; p.k1 = r.k1; p.ks = r.ks; p.vs = r.vs;
    p.v0 = r.v[0]; p.v1 = r.v[1]; p.v2 = r.v[2]; p.v3 = r.v[3];
    const int lane = tix() & 63;
    p.cs = gp(a.T.rope_cs)[pos * 128 + lane];
    p.sn = gp(a.T.rope_cs)[pos * 128 + 64 + lane];
    const GLB float *nq = (const GLB float *)plane(a, PL_Q_NORM, l), *nk = (const GLB float *)plane(a, PL_K_NORM, l);
    p.nq0 = nq[lane]; p.nq1 = nq[64 + lane];
    p.nk0 = nk[lane]; p.nk1 = nk[64 + lane];
}

// The Q/K/V words of head h's workgroup: q rows 128 h .. 128 h + 127, then the K and V rows
// (4096 .. 5119), into A.q, A.k, A.v
DEV bool attn_wait(const QxDArgs &a, uint32_t l, uint32_t ep, DLds &S, const Ctl &c) {
    const int h = blockIdx.x;
    const GLB uint64_t *qkv = gp(a.xch) + XO_QKV + (l & 1) * XN_QKV;
    return wait_xch2<2>(qkv, 1152, ep, reinterpret_cast<uint32_t *>(S.u.att.q), [h](int i) { return i < 128 ? 128 * h + i : 3968 + i; }, S, c);
}

// wave-level LDS hand-off: the wave's own earlier LDS writes are seen by its later reads
// (LDS instructions of a wave execute in order); this only keeps the compiler from
// reordering them
DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
DEV float wave_max_f(float v) {
    v = fmaxf(v, dppf<DPP_XOR1>(v)); v = fmaxf(v, dppf<DPP_XOR2>(v));
    v = fmaxf(v, dppf<DPP_ROR4>(v)); v = fmaxf(v, dppf<DPP_ROR8>(v));
    return fmaxf(fmaxf(rdlanef(v, 0), rdlanef(v, 16)), fmaxf(rdlanef(v, 32), rdlanef(v, 48)));
}

// ep: the QKV phase (the context goes out at ep + 1)
// rrow: the record row (slot * layers + l) of this layer's dumps, or -1
DEV void attention(const QxDArgs &a, uint32_t l, uint32_t pos, uint32_t ep, const AttnPre &pre, DLds &S, bool last, int rrow) {
    AttnS &A = S.u.att;
    const int tid = tix(), lane = tid & 63;
    const int w = wave_id();
    const int h = blockIdx.x, kvh = h >> 3;
    AttnW &W = A.w[w];
    const uint32_t n = pos + 1;
    // ---- the position's rows: waves 0..3 normalise and rotate k of kv head w (in place) and
    // take its largest magnitude; wave 4 normalises and rotates q and forms its digit planes
    // (lanes 0..15); waves 5..7 take the largest magnitudes of the four v heads
    if (w < 4) {
        float k0 = A.k[128 * w + lane], k1 = A.k[128 * w + 64 + lane];
        head_norm_rope_wave(k0, k1, pre.nk0, pre.nk1, pre.cs, pre.sn);
        A.k[128 * w + lane] = k0;
        A.k[128 * w + 64 + lane] = k1;
        const float mx = wave_max_f(fmaxf(int8_mag(k0), int8_mag(k1)));
        if (lane == 0) A.kmx[w] = mx;
    } else if (w > 4) {   // v heads 0, 1 (wave 5), 2 (wave 6), 3 (wave 7)
        const int j0 = w == 5 ? 0 : w - 4, j1 = w == 5 ? 1 : w - 4;
        const float v0 = A.v[128 * j0 + lane], v1 = A.v[128 * j0 + 64 + lane];
        const float v2 = A.v[128 * j1 + lane], v3 = A.v[128 * j1 + 64 + lane];
        const float m0 = wave_max_f(fmaxf(int8_mag(v0), int8_mag(v1)));
        const float m1 = wave_max_f(fmaxf(int8_mag(v2), int8_mag(v3)));
        if (lane == 0) { A.vmx[j0] = m0; A.vmx[j1] = m1; }
    } else {   // wave 4
        {
            float q0 = A.q[lane], q1 = A.q[64 + lane];
            head_norm_rope_wave(q0, q1, pre.nq0, pre.nq1, pre.cs, pre.sn);
            A.q[lane] = q0;
            A.q[64 + lane] = q1;
            wave_lds_sync();
            bool qfin = true;
            if (lane < 16) {
                float y[8];
                const float4 a0 = reinterpret_cast<const float4 *>(A.q)[2 * lane], a1 = reinterpret_cast<const float4 *>(A.q)[2 * lane + 1];
                y[0] = a0.x; y[1] = a0.y; y[2] = a0.z; y[3] = a0.w; y[4] = a1.x; y[5] = a1.y; y[6] = a1.z; y[7] = a1.w;
                float mx2 = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) { qfin = qfin && isfinite(y[i]); mx2 = fmaxf(mx2, fabsf(y[i])); }
                mx2 = fmaxf(mx2, dppf<DPP_XOR1>(mx2));
                mx2 = fmaxf(mx2, dppf<DPP_XOR2>(mx2));
                uint32_t h0, h1, m0, m1, l0, l1;
                float scq;
                digits8(y, isfinite(mx2) ? mx2 : 0.0f, h0, h1, m0, m1, l0, l1, scq);
                uint32_t *dd = A.qd + (lane >> 2) * DIG_STRIDE;
                const int q = lane & 3;
                *reinterpret_cast<uint2 *>(dd + 2 * q) = make_uint2(h0, h1);
                *reinterpret_cast<uint2 *>(dd + 8 + 2 * q) = make_uint2(m0, m1);
                *reinterpret_cast<uint2 *>(dd + 16 + 2 * q) = make_uint2(l0, l1);
                if (q == 0) dd[24] = __float_as_uint(scq);
            }
            const bool allfin = __ballot(!qfin) == 0;
            if (lane == 0) A.qok = allfin ? 1u : 0u;
        }
    }
    DMARK(l, 25);
    __syncthreads();
    DMARK(l, 21);
    const float kmx = fmaxf(fmaxf(A.kmx[0], A.kmx[1]), fmaxf(A.kmx[2], A.kmx[3]));
    const float vmx = fmaxf(fmaxf(A.vmx[0], A.vmx[1]), fmaxf(A.vmx[2], A.vmx[3]));
    const float kscale = int8_scale(kmx), vscale = int8_scale(vmx);
    const bool qok = A.qok != 0u;
    // the codes of the workgroup's kv head for the position, by the wave whose block holds it
    const int wpos = (int)((pos & 127u) >> 4);
    if (w == wpos) {
        W.kc[lane] = int8_code(A.k[128 * kvh + lane], kscale);
        W.kc[64 + lane] = int8_code(A.k[128 * kvh + 64 + lane], kscale);
        W.vc[lane] = int8_code(A.v[128 * kvh + lane], vscale);
        W.vc[64 + lane] = int8_code(A.v[128 * kvh + 64 + lane], vscale);
    }
    if (h == 0) {   // the position's rows into the cache, coherent (later steps read them): wave w
        // stores the K row of kv head w (w < 4) or the V row of kv head w - 4
        const int j = w & 3;
        const float *src = w < 4 ? A.k : A.v;
        const float sc = w < 4 ? kscale : vscale;
        int8_t *dst = (w < 4 ? A.kq : A.vq) + 128 * j;
        dst[lane] = int8_code(src[128 * j + lane], sc);
        dst[64 + lane] = int8_code(src[128 * j + 64 + lane], sc);
        wave_lds_sync();
        const uint32_t slot = l * a.ctx + pos;   // layers * ctx * 512 < 2^32
        GLB uint32_t *row = (GLB uint32_t *)gpw(w < 4 ? a.kc : a.vc) + slot * 128 + 32 * j;
        if (lane < 32) st_coherent(row + lane, reinterpret_cast<const uint32_t *>(dst)[lane]);
        if (w == 0 && lane == 0) {
            st_coherent((GLB uint32_t *)gpw(a.ks) + slot, __float_as_uint(kscale));
            st_coherent((GLB uint32_t *)gpw(a.vs) + slot, __float_as_uint(vscale));
        }
    }
    wave_lds_sync();
    DMARK(l, 22);
    // ---- positions 128 i + 16 w + j: scores (a quad per position), online softmax, context
    const int q4 = lane & 3, jq = lane >> 2, p4 = lane >> 4, dg = lane & 15;
    Dig d;
    load_dig(A.qd, q4, d);
    // scores and the running maximum in double (planted x1e6 channels make scores large
    // enough that an f32 difference s - m loses the 1e-5 bar); the exponentials in f32 of
    // that double difference (a double exp's polynomial constants spill the layer loop)
    const double inv_sqrt_hd = 1.0 / a.sqrt_hd;
    double m = -INFINITY, lsum = 0.0;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    AttnRows cur, nxt;
    cur.k0 = pre.k0; cur.k1 = pre.k1; cur.ks = pre.ks; cur.vs = pre.vs;
    cur.v[0] = pre.v0; cur.v[1] = pre.v1; cur.v[2] = pre.v2; cur.v[3] = pre.v3;
    for (uint32_t t0 = 0; t0 < n; t0 += 128) {
        if (t0 + 128 < n) attn_rows(a, l, pos, t0 + 128, nxt);   // the next block's rows, ahead
        const uint32_t tq = t0 + 16u * w + (uint32_t)jq;
        uint32_t kw[8];
        float ksc = cur.ks, vsc = cur.vs;
        kw[0] = cur.k0.x; kw[1] = cur.k0.y; kw[2] = cur.k0.z; kw[3] = cur.k0.w;
        kw[4] = cur.k1.x; kw[5] = cur.k1.y; kw[6] = cur.k1.z; kw[7] = cur.k1.w;
        if (tq == pos) {
            const uint4 *pk = reinterpret_cast<const uint4 *>(W.kc + 32 * q4);
            const uint4 x0 = pk[0], x1 = pk[1];
            kw[0] = x0.x; kw[1] = x0.y; kw[2] = x0.z; kw[3] = x0.w; kw[4] = x1.x; kw[5] = x1.y; kw[6] = x1.z; kw[7] = x1.w;
            ksc = kscale;
            vsc = vscale;
        }
        int aH = 0, aM = 0, aL = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            aH = sdot4s(kw[i], d.h[i], aH, i == 0);
            aM = sdot4s(kw[i], d.m[i], aM, i == 0);
            aL = sdot4s(kw[i], d.l[i], aL, i == 0);
        }
        double sq = (double)(combine(aH, aM, aL) * d.s);
        sq += dppd<DPP_XOR1>(sq);
        sq += dppd<DPP_XOR2>(sq);
        double sc = qok ? sq * (double)ksc * inv_sqrt_hd : 0.0;
        if (!isfinite(sc)) sc = 0.0;
        const bool valid = tq < n;
        const double mi = wave_max_d(valid ? sc : -INFINITY);
        if (mi != -INFINITY) {   // wave-uniform: the block holds some of the wave's positions
            const double mn = fmax(m, mi);
            const float f = expf((float)(m - mn));   // 0 on the first block with positions (m = -inf)
            const float e = valid ? expf((float)(sc - mn)) : 0.0f;
            lsum = lsum * (double)f + wave_total_f(q4 == 0 ? e : 0.0f);
            if (q4 == 0) W.p[jq] = e * vsc;
            wave_lds_sync();
            const float ff = f;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] *= ff;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t jv = 4u * i + (uint32_t)p4, tv = t0 + 16u * w + jv;
                const float pv = W.p[jv];
                u32x2 x = cur.v[i];
                if (tv == pos) x = reinterpret_cast<const u32x2 *>(W.vc)[dg];
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const int8_t vb = (int8_t)((((b < 4) ? x.x : x.y) >> (8 * (b & 3))) & 255u);
                    acc[b] = fmaf(pv, (float)vb, acc[b]);
                }
            }
            wave_lds_sync();   // W.p is rewritten by the next block
            m = mn;
        }
        if (t0 + 128 < n) cur = nxt;
    }
    DMARK(l, 23);
    // the wave's four 16-lane rows (positions 4 i + p4) summed by the wave itself, so the
    // merge below reads one partial per wave
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = rows4_sum(acc[i]);
    if (p4 == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) A.ctx[w][8 * dg + i] = acc[i];
    }
    if (lane == 0) { A.m[w] = m; A.l[w] = lsum; }
    __syncthreads();
    DMARK(l, 24);
    if (tid < 128) {
        double M = A.m[0];
#pragma unroll
        for (int v = 1; v < NWV; ++v) M = fmax(M, A.m[v]);
        // lane v < 8 forms wave v's factor exp(m_v - M); every lane then reads the eight
        const double mv = A.m[lane & 7];
        const double fl = mv == -INFINITY ? 0.0 : (double)expf((float)(mv - M));   // (f32, as the block loop)
        double fw[NWV], L = 0.0;
#pragma unroll
        for (int v = 0; v < NWV; ++v) { fw[v] = rdlaned(fl, v); L += fw[v] * A.l[v]; }
        if (!isfinite(L) || L <= 0.0) L = 1.0;
        const double invL = 1.0 / L;
        float o = 0.0f;
#pragma unroll
        for (int v = 0; v < NWV; ++v) {
            o = fmaf((float)(fw[v] * invL), A.ctx[v][tid], o);
        }
        xstf(gpw(a.xch) + XO_CX + (l & 1) * XN_CX + 128 * h + tid, ep + 1, o);   // the CX phase
        if (rrow >= 0 && a.d_wsum && tid == 0) {   // the head's sum of normalised weights (the state loop's softmax_sum)
            double ws = 0.0;
#pragma unroll
            for (int v = 0; v < NWV; ++v) ws += (fw[v] * invL) * A.l[v];
            gpw(a.d_wsum)[(uint32_t)rrow * 32 + h] = ws;
        }
    }
    __syncthreads();   // the union is reused by the next stage
}

// ---------------------------------------------------------------- attention by chunk (stage A, long context)
// The same attention (reference src/qx_format.c:5051-5196) spread over every workgroup once
// the cache is long: with n = pos + 1 positions in chunks of cs = 32 positions (n <= 2048) or
// 64 (nch <= 64 chunks either way), workgroup w < 4 nch takes kv head g = w % 4 and chunk
// c = w / 4 for all eight q heads that share g (wave v: q head 8 g + v), so each chunk's K and V
// rows are read once, into LDS in stage Q (dma_chunk), for eight heads.  A wave scores the
// chunk's positions (a quad per position, rounds of 16), takes one maximum and one
// exponential per lane, and sums the
// weighted V codes (lane: 4 dimensions, odd or even positions).  Its partial result - the
// chunk's maximum score m_c, its sum of exp(s - m_c) and the f32 context sums - is published
// as 8 records of 16 dimensions.  Then workgroup w merges q head w / 8, dimensions
// 16 (w % 8) .. over the chunks: ctx[d] = sum_c (float)(exp(m_c - M) / L) acc_c[d],
// L = sum_c exp(m_c - M) l_c, the formula of the per-wave merge in attention().
// The chunk holding the position (c = nch - 1) quantizes its kv head's K and V rows of the
// position (scales over all 512 values of the row) and stores them in the cache.
DEV uint32_t pack_codes4(const float *v, float sc) {
    return (uint32_t)(uint8_t)int8_code(v[0], sc) | ((uint32_t)(uint8_t)int8_code(v[1], sc) << 8) |
           ((uint32_t)(uint8_t)int8_code(v[2], sc) << 16) | ((uint32_t)(uint8_t)int8_code(v[3], sc) << 24);
}
DEV double dbl_words(uint32_t hi, uint32_t lo) { return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo)); }
// positions per chunk: QXD_CHUNK_S up to QXD_CHUNK_S_MAXN cached positions, QXD_CHUNK beyond
// (at most QXG_MAX_CTX / QXD_CHUNK = 64 chunks either way)
DEV uint32_t chunk_size(uint32_t pos) { return pos + 1 <= QXD_CHUNK_S_MAXN ? QXD_CHUNK_S : QXD_CHUNK; }
DEV uint32_t chunk_count(uint32_t pos) { const uint32_t cs = chunk_size(pos); return (pos + cs) / cs; }   // ceil((pos + 1) / cs)
DEV ChunkRows &chunk_rows(DLds &S) {
    static_assert(sizeof(ChunkRows) <= sizeof(S.u.m.dn), "a chunk's rows fit the down-row area");
    static_assert(sizeof(AttnK) <= offsetof(decltype(S.u.m), dn), "the chunk workgroup's scratch stays clear of its rows");
    return *reinterpret_cast<ChunkRows *>(&S.u.m.dn[0][0]);
}

// Stage Q of a chunk workgroup (w < 4 nch): its chunk's cached rows (positions c0 .. c0 + cs - 1,
// clamped below pos) and scales to LDS; wave v copies rows rpw v .. rpw v + rpw - 1 of K and of
// V (rpw = cs / 8 rows, 8 lanes a row; the other lanes idle).
DEV void dma_chunk(const QxDArgs &a, uint32_t l, uint32_t pos, DLds &S) {
    const int lane = tix() & 63, w = wave_id();
    const uint32_t cs = chunk_size(pos), rpw = cs / 8u;
    const uint32_t g = blockIdx.x & 3u, c0 = (blockIdx.x >> 2) * cs;
    const uint32_t lastc = pos > 0 ? pos - 1 : 0u, base = l * a.ctx;
    ChunkRows &C = chunk_rows(S);
    if ((uint32_t)(lane >> 3) < rpw) {
        const uint32_t t = min(c0 + rpw * w + (uint32_t)(lane >> 3), lastc);
        const uint32_t off = (base + t) * 512 + 128 * g + 16 * (lane & 7);   // layers * ctx * 512 < 2^32
        dma16_kv(gp(reinterpret_cast<const uint8_t *>(a.kc)), off, C.k[rpw * w]);
        dma16_kv(gp(reinterpret_cast<const uint8_t *>(a.vc)), off, C.v[rpw * w]);
    }
    if (w < 2 && (uint32_t)lane < cs) {
        const uint32_t ts = min(c0 + (uint32_t)lane, lastc);
        dma4_kv(gp(reinterpret_cast<const uint8_t *>(w == 0 ? a.ks : a.vs)), (base + ts) * 4, w == 0 ? C.ks : C.vs);
    }
}

// ep: the QKV phase (the partial results go out at ep + 1).  The chunk's rows are in LDS once
// the Q/K/V poll has returned (its loads complete after the earlier copies).
DEV bool attention_chunk_part(const QxDArgs &a, uint32_t l, uint32_t pos, uint32_t ep, DLds &S, const Ctl &ctl, bool last) {
    (void)last;
    constexpr uint32_t MAXCH = QXG_MAX_CTX / QXD_CHUNK;
    GLB uint64_t *const X = gpw(a.xch);
    const uint32_t n = pos + 1, nch = chunk_count(pos), csz = chunk_size(pos), par = l & 1;
    AttnK &A = S.u.atk;
    ChunkRows &C = chunk_rows(S);
    const int g = blockIdx.x & 3;
    const uint32_t ch = blockIdx.x >> 2, c0 = ch * csz;
    const bool own = ch + 1 == nch;   // the chunk holding the position (workgroup-uniform)
    const int tid = tix(), lane = tid & 63, w = wave_id();
    const double cs = gp(a.T.rope_cs)[pos * 128 + lane], sn = gp(a.T.rope_cs)[pos * 128 + 64 + lane];
    const GLB float *nqp = (const GLB float *)plane(a, PL_Q_NORM, l), *nkp = (const GLB float *)plane(a, PL_K_NORM, l);
    const float nq0 = nqp[lane], nq1 = nqp[64 + lane], nk0 = nkp[lane], nk1 = nkp[64 + lane];
    // q of heads 8 g .. 8 g + 7 (words 1024 g ..), then the K and V rows (4096 .. 5119)
    const GLB uint64_t *qkv = X + XO_QKV + par * XN_QKV;
    if (!wait_xch2<2>(qkv, 2048, ep, reinterpret_cast<uint32_t *>(A.q[0]), [g](int i) { return i < 1024 ? 1024 * g + i : 3072 + i; },
                      S, ctl))
        return false;
    DMARK(l, 3);
    // ---- wave v: q head 8 g + v normalised, rotated, as digit planes; the position's chunk
    // also the K heads (waves 0..3, in place) and the V maxima (waves 4..7)
    {
        float q0 = A.q[w][lane], q1 = A.q[w][64 + lane];
        head_norm_rope_wave(q0, q1, nq0, nq1, cs, sn);
        A.q[w][lane] = q0;
        A.q[w][64 + lane] = q1;
        wave_lds_sync();
        bool qfin = true;
        if (lane < 16) {
            float y[8];
            const float4 a0 = reinterpret_cast<const float4 *>(A.q[w])[2 * lane], a1 = reinterpret_cast<const float4 *>(A.q[w])[2 * lane + 1];
            y[0] = a0.x; y[1] = a0.y; y[2] = a0.z; y[3] = a0.w; y[4] = a1.x; y[5] = a1.y; y[6] = a1.z; y[7] = a1.w;
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) { qfin = qfin && isfinite(y[i]); mx = fmaxf(mx, fabsf(y[i])); }
            mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
            mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
            uint32_t h0, h1, m0, m1, l0, l1;
            float scq;
            digits8(y, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, scq);
            uint32_t *dd = A.qd[w] + (lane >> 2) * DIG_STRIDE;
            const int q = lane & 3;
            *reinterpret_cast<uint2 *>(dd + 2 * q) = make_uint2(h0, h1);
            *reinterpret_cast<uint2 *>(dd + 8 + 2 * q) = make_uint2(m0, m1);
            *reinterpret_cast<uint2 *>(dd + 16 + 2 * q) = make_uint2(l0, l1);
            if (q == 0) dd[24] = __float_as_uint(scq);
        }
        const bool allfin = __ballot(!qfin) == 0;
        if (lane == 0) A.qok[w] = allfin ? 1u : 0u;
    }
    if (own) {
        if (w < 4) {
            float k0 = A.k[128 * w + lane], k1 = A.k[128 * w + 64 + lane];
            head_norm_rope_wave(k0, k1, nk0, nk1, cs, sn);
            A.k[128 * w + lane] = k0;
            A.k[128 * w + 64 + lane] = k1;
            const float mx = wave_max_f(fmaxf(int8_mag(k0), int8_mag(k1)));
            if (lane == 0) A.kmx[w] = mx;
        } else {
            const int j = w - 4;
            const float mx = wave_max_f(fmaxf(int8_mag(A.v[128 * j + lane]), int8_mag(A.v[128 * j + 64 + lane])));
            if (lane == 0) A.vmx[j] = mx;
        }
    }
    __syncthreads();
    DMARK(l, 21);
    if (own) {
        // the position's codes of kv head g (wave 0 K, wave 1 V, 4 per lane) replace the copied
        // row in its chunk slot (pos - c0; the copy held position pos - 1 there), and go to the
        // cache, coherent (later steps read them)
        const float kscale = int8_scale(fmaxf(fmaxf(A.kmx[0], A.kmx[1]), fmaxf(A.kmx[2], A.kmx[3])));
        const float vscale = int8_scale(fmaxf(fmaxf(A.vmx[0], A.vmx[1]), fmaxf(A.vmx[2], A.vmx[3])));
        const uint32_t up = pos - c0;
        if (w < 2 && lane < 32) {
            const uint32_t word = pack_codes4((w == 0 ? A.k : A.v) + 128 * g + 4 * lane, w == 0 ? kscale : vscale);
            reinterpret_cast<uint32_t *>(w == 0 ? C.k[up] : C.v[up])[lane] = word;
            const uint32_t slot = l * a.ctx + pos;   // layers * ctx * 512 < 2^32
            GLB uint32_t *row = (GLB uint32_t *)gpw(w == 0 ? a.kc : a.vc) + slot * 128 + 32 * g;
            st_coherent(row + lane, word);
            if (lane == 0) {
                (w == 0 ? C.ks : C.vs)[up] = w == 0 ? kscale : vscale;
                if (g == 0) st_coherent((GLB uint32_t *)gpw(w == 0 ? a.ks : a.vs) + slot, __float_as_uint(w == 0 ? kscale : vscale));
            }
        }
        __syncthreads();
    }
    DMARK(l, 22);
    // ---- scores of positions c0 + 16 i + jq (a quad per position; lane q4 takes dims 32 q4 ..)
    const int q4 = lane & 3, jq = lane >> 2;
    Dig d;
    load_dig(A.qd[w], q4, d);
    const bool qok = A.qok[w] != 0u;
    const double inv_sqrt_hd = 1.0 / a.sqrt_hd;
    double sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t u = 16u * i + (uint32_t)jq, t = c0 + u;
        const uint4 x0 = *reinterpret_cast<const uint4 *>(C.k[u] + 32 * q4), x1 = *reinterpret_cast<const uint4 *>(C.k[u] + 32 * q4 + 16);
        const uint32_t kw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float ksc = C.ks[u];
        int aH = 0, aM = 0, aL = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            aH = sdot4s(kw[k], d.h[k], aH, k == 0);
            aM = sdot4s(kw[k], d.m[k], aM, k == 0);
            aL = sdot4s(kw[k], d.l[k], aL, k == 0);
        }
        double sq = (double)(combine(aH, aM, aL) * d.s);
        sq += dppd<DPP_XOR1>(sq);
        sq += dppd<DPP_XOR2>(sq);
        double v = qok ? sq * (double)ksc * inv_sqrt_hd : 0.0;
        if (!isfinite(v)) v = 0.0;
        sc[i] = u < csz && t < n ? v : -INFINITY;   // (rows past a 32-position chunk are stale LDS)
    }
    const double m = wave_max_d(fmax(fmax(sc[0], sc[1]), fmax(sc[2], sc[3])));
    // one exponential per lane: lane (jq, q4) weighs position c0 + 16 q4 + jq
    double ss = sc[0];
    if (q4 == 1) ss = sc[1];
    if (q4 == 2) ss = sc[2];
    if (q4 == 3) ss = sc[3];
    const uint32_t u = 16u * q4 + (uint32_t)jq;
    const bool uvalid = u < csz && c0 + u < n;
    const float vsel = C.vs[u];
    // the exponentials of the chunked path in f32 (arguments <= 0, relative error ~1e-7: far
    // inside the 1e-5 bar; a double exp is a long dependent chain)
    const double e = uvalid ? (double)expf((float)(ss - m)) : 0.0;
    const double lsum = wave_total_d(e);
    A.p[w][u] = uvalid ? (float)(e * (double)vsel) : 0.0f;   // (a clamped row's scale may be unset)
    wave_lds_sync();
    DMARK(l, 23);
    // ---- context sums: lane (p4 = lane / 16, dims 8 dg ..) over positions 4 j + p4, then the
    // four position groups added (xor 16, then xor 32: the same order in every lane)
    const int p4 = lane >> 4, dg = lane & 15;
    float acc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = 0.0f;
#pragma unroll 4
    for (int j = 0; j < (int)(csz / 4u); ++j) {
        const uint32_t uu = 4u * j + (uint32_t)p4;
        const float pv = A.p[w][uu];
        const uint2 x = *reinterpret_cast<const uint2 *>(C.v[uu] + 8 * dg);
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[b] = fmaf(pv, (float)(int8_t)((((b < 4) ? x.x : x.y) >> (8 * (b & 3))) & 255u), acc[b]);
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = rows4_sum_pairs(acc[b]);
    // ---- the wave's partial result, 8 records of 16 dimensions: lanes 0..31 the context sums
    // (lane (p4 < 2, dg): dims 8 dg + 4 p4 .. of record dg / 2), lanes 32..63 the maximum and
    // the denominator
    {
        const uint32_t hq = 8u * g + (uint32_t)w;
        GLB uint64_t *pt = gpw(a.xpart) + par * XN_PT;
        if (lane < 32) {
            GLB uint64_t *rec = pt + ((hq * 8u + (uint32_t)(dg >> 1)) * MAXCH + ch) * QXD_PREC + 8 * (dg & 1) + 4 * p4;
            const uint32_t hi = p4 ? 0xffffffffu : 0u;   // (a bit select: a lane-dependent index would go through scratch)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                xst(rec + b, ep + 1, (__float_as_uint(acc[4 + b]) & hi) | (__float_as_uint(acc[b]) & ~hi));
        } else {
            const int r = (lane - 32) >> 2, k = lane & 3;   // record r, word 16 + k
            const uint64_t bits = (uint64_t)__double_as_longlong(k < 2 ? m : lsum);
            GLB uint64_t *rec = pt + ((hq * 8u + (uint32_t)r) * MAXCH + ch) * QXD_PREC + 16 + k;
            xst(rec, ep + 1, (k & 1) ? (uint32_t)bits : (uint32_t)(bits >> 32));
        }
    }
    DMARK(l, 24);
    __syncthreads();   // the union is reused by the merge
    return true;
}

// Every workgroup: q head wgi / 8, dimensions 16 (wgi % 8) .. merged over the chunks, published
// as its context words.  ep: the partial results' phase (the context goes out with it too).
DEV bool attention_merge(const QxDArgs &a, uint32_t l, uint32_t pos, uint32_t ep, DLds &S, const Ctl &ctl, bool last, int rrow) {
    (void)last;
    constexpr uint32_t MAXCH = QXG_MAX_CTX / QXD_CHUNK;
    static_assert(4 * MAXCH <= NWG && 32 * 8 == NWG, "one workgroup per (kv head, chunk) and per (q head, 16 dims)");
    GLB uint64_t *const X = gpw(a.xch);
    const uint32_t nch = chunk_count(pos), par = l & 1;
    const int lane = tix() & 63, w = wave_id();
    const uint32_t h = blockIdx.x >> 3, dgm = blockIdx.x & 7u;
    uint32_t *rw = S.u.m.vin;                                           // nch records of QXD_PREC words
    float *wt = reinterpret_cast<float *>(S.u.m.vin) + 2048;            // per chunk: (float)(exp(m_c - M) / L)
    const GLB uint64_t *src = gpw(a.xpart) + par * XN_PT + (h * 8u + dgm) * MAXCH * QXD_PREC;
    QXD_SLEEP(QXD_SLEEP_MG);
    if (!wait_xch2<2>(src, (int)(QXD_PREC * nch), ep, rw, Ident(), S, ctl)) return false;
    DMARK(l, 25);
    if (w == 0) {   // wave 0 alone: lane c forms chunk c's factor, then lane (cg, d) sums chunks cg + 4 k
        double mc = -INFINITY, lc = 0.0;
        if ((uint32_t)lane < nch) {
            mc = dbl_words(rw[QXD_PREC * lane + 16], rw[QXD_PREC * lane + 17]);
            lc = dbl_words(rw[QXD_PREC * lane + 18], rw[QXD_PREC * lane + 19]);
        }
        const double M = wave_max_d(mc);
        const double f = mc == -INFINITY ? 0.0 : (double)expf((float)(mc - M));
        double L = wave_total_d(f * lc);
        if (!isfinite(L) || L <= 0.0) L = 1.0;
        const double invL = 1.0 / L;
        wt[lane] = (float)(f * invL);
        if (rrow >= 0 && a.d_wsum) {   // the head's sum of normalised weights (the state loop's softmax_sum)
            const double ws = wave_total_d((f * invL) * lc);
            if (dgm == 0 && lane == 0) gpw(a.d_wsum)[(uint32_t)rrow * 32 + h] = ws;
        }
        wave_lds_sync();
        const int dd = lane & 15, cg = lane >> 4;
        float o = 0.0f;
        for (uint32_t cc = (uint32_t)cg; cc < nch; cc += 4) o = fmaf(wt[cc], __uint_as_float(rw[QXD_PREC * cc + dd]), o);
        o = rows4_sum_pairs(o);
        if (lane < 16) xstf(X + XO_CX + par * XN_CX + 128 * h + 16 * dgm + lane, ep, o);   // the CX phase
    }
    DMARK(l, 39);
    __syncthreads();   // the union is reused by the next stage
    return true;
}

// ---------------------------------------------------------------- head
// Output RMSNorm + Q6_K head (src/qx_format.c:3554-3738) over the digits in S.dig: group g
// is rows R g .. R g + R - 1; workgroup w's groups are w + 256 j, its waves taking them in
// turn (S.u.hd.next, zeroed before the call).  A pass's R interleaved rows
// (R * 105 16-byte chunks, contiguous) come in with HEAD_NI full-width loads and go to the
// wave's LDS region; the next pass's loads are issued before this pass's dots.  Lane (b, ib)
// then reads its sub-block's ql, qh, scale pair and d from LDS.  Returns the workgroup's best
// (logit desc, index asc) through bv/bi (uniform); non-finite logits set *nonfin.
template <bool H1>
DEV void head_rows(const QxDArgs &a, DLds &S, bool fin, float &bv, uint32_t &bi, bool &nonfin, uint32_t rslot) {
    constexpr int R = HEAD_R;
    const int lane = tix() & 63, wave = wave_id();
    const int b = lane >> 3, ib = lane & 7, hh = ib >> 2, k = ib & 3;
    Dig g;
    load_dig(S.dig, lane, g);
    const Q6Bias bias = q6_bias(g);
    float best = -INFINITY;
    uint32_t besti = 0xffffffffu;
    bool nf = false;
    const uint32_t groups = (a.vocab + R - 1) / R;
    const uint64_t hb = uni64((uint64_t)a.h_il);
    GLB float *lg = a.logits ? gpw(a.logits) + (uint64_t)rslot * a.vocab : nullptr;
    uint8_t *rows = S.u.hd.rows[wave];
    u32x4 v[HEAD_NI];
    auto issue = [&](uint32_t p) {
#pragma unroll
        for (int i = 0; i < HEAD_NI; ++i) {
            const uint32_t c = 64 * i + lane, rr = c / 105u, cc = c - 105u * rr;
            const uint32_t row = c < (uint32_t)R * 105u ? min(R * p + rr, a.vocab - 1) : min(R * p, a.vocab - 1);
            const uint32_t ch = c < (uint32_t)R * 105u ? cc : 0u;
            v[i] = __builtin_nontemporal_load((const GLB u32x4 *)(hb + (uint64_t)row * QXD_HEAD_ROW + 16 * ch));
        }
    };
    // the workgroup's groups blockIdx.x + NWG j, j taken in turn from an LDS counter: the two
    // waves of a SIMD are not served equally (the older one issues first), so with fixed
    // shares waves 4..7 finished 13 us after waves 0..3, alone and with half the loads in
    // flight.  Each wave's groups still ascend.
    auto take = [&]() -> uint32_t {
        uint32_t j = 0u;
        if (lane == 0) j = __hip_atomic_fetch_add(&S.u.hd.next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return blockIdx.x + NWG * (uint32_t)__builtin_amdgcn_readfirstlane((int)j);
    };
    uint32_t p = take();
    if (p < groups) issue(p);
    while (p < groups) {
#pragma unroll
        for (int i = 0; i < HEAD_NI; ++i) *reinterpret_cast<u32x4 *>(rows + 1024 * i + 16 * lane) = v[i];
        wave_lds_sync();
        const uint32_t pn = take();
        if (pn < groups) issue(pn);   // the next pass's rows, in flight during the dots
        float part[R], out[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const uint8_t *r = rows + rr * QXD_HEAD_ROW;
            const uint32_t lo = b * 128 + 64 * hh + 32 * (k & 1), ho = 1024 + b * 64 + 32 * hh;
            const uint4 l0 = *reinterpret_cast<const uint4 *>(r + lo), l1 = *reinterpret_cast<const uint4 *>(r + lo + 16);
            const uint4 h0 = *reinterpret_cast<const uint4 *>(r + ho), h1 = *reinterpret_cast<const uint4 *>(r + ho + 16);
            const uint32_t so = 1536 + b * 16 + 8 * hh + 2 * k;
            const int s0 = (int8_t)r[so], s1 = (int8_t)r[so + 1];
            const uint32_t d16 = *reinterpret_cast<const uint16_t *>(r + 1664 + 2 * b);
            part[rr] = dot_q6<H1>(l0, l1, h0, h1, s0, s1, d16, ib, g, bias);
        }
        wave_lds_sync();   // the rows are rewritten by the next pass
        rows_reduce<R>(part, out, lane);
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const uint32_t r = R * p + rr;
            if (r < a.vocab) {
                const float val = out[rr];
                if (!fin || !isfinite(val)) nf = true;
                if (lg && lane == rr) lg[r] = val;
                if (val > best) { best = val; besti = r; }   // rows ascend: ties keep the lower index
            }
        }
        p = pn;
    }
    bv = best;
    bi = besti;
    nonfin = nf;
}

// total order of the argmax: larger value, then lower index (NaN below every number)
DEV bool better(float v, uint32_t i, float bv, uint32_t bi) { return v > bv || (v == bv && i < bi); }

}  // namespace

// ================================================================= kernel
// The decode steps; CHUNKED: stage A by kv head and chunk (every step of the launch at
// n = pos + 1 >= att_split_min), else the 32 q-head workgroups' walk.  Two kernels, so neither
// carries the other's stage A code in its layer loop (the host splits a launch at the threshold).
template <bool CHUNKED, bool Q8>
DEV void decode_steps(const QxDArgs &args) {
    __shared__ DLds S;
#ifdef QXD_TRACE
    if (threadIdx.x < 5 * 40) qxd_tl[threadIdx.x / 40][threadIdx.x % 40] = 0ull;
#endif
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
        if (tid < 4) { S.sub[tid] = 0u; S.sublo[tid] = 0u; }   // the tags start above 0
        if (tid < NWV) S.bpar[tid] = 0u;
        if (tid == 0) S.fail = 0u;
    }
    WQ wq;
    WO wo;
    if (wg >= QXG_HEADS) load_wq(a, 0, wq, S.wq[wave_id()]);
    load_wr(a, 0, wo);
    uint32_t token = 0;
    __syncthreads();
    GLB uint64_t *const X = gpw(a.xch);
    for (uint32_t step = 0; step < a.steps; ++step) {
        const uint32_t pos = a.pos0 + step;
        const uint32_t ep_step = a.ep0 + step * phases + 1;
        const bool head_step = a.force_head || step + 1 >= a.n_prompt;
        const bool last = step + 1 == a.steps;
        const bool rec = last || a.rec_all != 0u;                // this step's dumps are written
        const uint32_t rslot = a.rec_all ? a.rec_base + step : 0u;   // ... at this record slot
        constexpr bool chunked = CHUNKED;
        if (step < a.n_prompt) token = gp(a.tokens)[step];
        if (a.d_time && wg == 0 && tix() == 0) gpw(a.d_time)[rslot] = __builtin_amdgcn_s_memrealtime();
        // embedding row of the token (reference src/qx_format.c:3759-3793), decoded by every
        // workgroup into its copy of x
        if (tix() < 256) embed_q4k_row((const uint8_t *)(gp(a.emb) + (uint64_t)token * a.emb_row), S.xs);
        __syncthreads();
        for (uint32_t l = 0; l < L; ++l) {
            // values loaded and used within one layer (declared here, they are not carried)
            AttnPre ap;
            float4 wm0, wm1;
            float fnw[8];
            const uint32_t ep = ep_step + 5 * l;   // + 0 X, + 1 QKV, + 2 CX, + 3 XP/LG, + 4 H/WT
            const uint32_t par = l & 1;
            const uint32_t rrow = rslot * L + l;            // the record row of this layer's dumps
            const uint32_t ln = l + 1 < L ? l + 1 : 0u;   // after the last layer: layer 0 of the next step
            // the next layer's rows are prefetched in this layer, except after the last layer of
            // a head step (layer 0's come in after the argmax exchange) or of the launch's last step
            const bool pre = l + 1 < L || !(head_step || last);
            // ---------------------------------------------------------- stage Q
            double a_part = 0.0;   // router x-part of expert wg (workgroups < E)
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                DMARK(l, 0);
                // x, and its sum of squares for the attention RMSNorm (reference
                // src/qx_format.c:3358-3371, a double sum) from each thread's 4 polled values:
                // the poll's barrier publishes the waves' sums with x (layer 0: the embedding,
                // already in LDS)
                {
                    double ssq = 0.0;
                    bool okx = true;
                    if (l > 0) {
                        QXD_SLEEP(QXD_SLEEP_X);
                        okx = poll_pairs<2>(X + XO_X + par * XN_X, 2048, ep, reinterpret_cast<uint32_t *>(S.xs), Ident(), ctl, &ssq);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) ssq += (double)S.xs[4 * tid + i] * (double)S.xs[4 * tid + i];
                    }
                    ssq = wave_total_d(ssq);
                    if (lane == 0) S.red[wave] = ssq;
                    if (block_any(!okx, S)) return;
                }
                DMARK(l, 1);
                wait_loads();   // the Q/K/V rows in LDS (issued a stage or more ago; nothing later is outstanding)
                // attention workgroups (no Q/K/V rows of their own): the cached K/V rows they
                // attend to, arriving while the other workgroups make the Q/K/V rows
                const bool mk = wg >= QXG_HEADS;
                if (!mk) {
                    if (!chunked) attn_prefetch(a, l, pos, ap);
                    load_o(a, l, wo, S.wo[wave_id()]);   // (the others load them after their rows)
                }
                if (chunked && (uint32_t)wg < 4u * chunk_count(pos)) dma_chunk(a, l, pos, S);
                DMARK(l, 32);
                // the normalised input's digits; the attn-norm weights came with the Q/K/V rows
                double inv = 1.0;
                bool fin = true;
                {
                    // router x-part: sum_i W[e,i] w_i x_i over values 4 tid .. 4 tid + 3
                    if ((uint32_t)wg < E) {
                        const float4 x4 = reinterpret_cast<const float4 *>(S.xs)[tid];
                        a_part = (double)wo.wr.x * (double)wo.fw.x * (double)x4.x + (double)wo.wr.y * (double)wo.fw.y * (double)x4.y +
                                 (double)wo.wr.z * (double)wo.fw.z * (double)x4.z + (double)wo.wr.w * (double)wo.fw.w * (double)x4.w;
                    }
                    DMARK(l, 33);
                    const double tot = ((S.red[0] + S.red[1]) + (S.red[2] + S.red[3])) + ((S.red[4] + S.red[5]) + (S.red[6] + S.red[7]));
                    inv = 1.0 / sqrt(tot / 2048.0 + 1.0e-6);
                }
                if (mk && tid < 256) {
                    float y[8];
                    const float nw8[8] = {wq.nw0.x, wq.nw0.y, wq.nw0.z, wq.nw0.w, wq.nw1.x, wq.nw1.y, wq.nw1.z, wq.nw1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) y[i] = (float)((double)S.xs[8 * tid + i] * inv) * nw8[i];
                    if constexpr (Q8) {   // (waves 0..3 whole)
#pragma unroll
                        for (int i = 0; i < 8; ++i) fin = fin && isfinite(y[i]);
                        store_q8(y, tid, S.dig);
                    } else {
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
                }
                if ((uint32_t)wg < E) {
                    a_part = wave_total_d(a_part);
                    if (lane == 0) S.red[NWV + wave] = a_part;
                }
                DMARK(l, 34);
                const bool ok = !block_any(!fin, S);
                if (Q8 && !ok && tid == 0) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_INPUT;   // (src/qx_format.c:3906)
                DMARK(l, 13);
                if ((uint32_t)wg < E)
                    a_part = ((S.red[NWV + 0] + S.red[NWV + 1]) + (S.red[NWV + 2] + S.red[NWV + 3])) +
                             ((S.red[NWV + 4] + S.red[NWV + 5]) + (S.red[NWV + 6] + S.red[NWV + 7]));
                if (mk) {
                    Dig g;
                    load_dig(S.dig, lane, g);
                    float part[4], out[4];
                    {
                        const uint4(*lq)[64] = S.wq[wave_id()];
                        part[0] = dot_iq4<Q8, true>(lq[0][lane], wq.m[0], ib, g);
                        part[1] = dot_iq4<Q8, true>(lq[1][lane], wq.m[1], ib, g);
                        part[2] = dot_iq4<Q8, true>(lq[2][lane], wq.m[2], ib, g);
                    }
                    part[3] = 0.0f;
                    rows_reduce<4>(part, out, lane);
                    // gather the workgroup's 24 rows, then one store: stacked rows 24 (wg - 32) ..
#pragma unroll
                    for (int r = 0; r < 3; ++r)
                        if (lane == r) S.outw[3 * wave + r] = (ok && isfinite(out[r])) ? out[r] : 0.0f;
                }
                __syncthreads();
                if (mk && tid < 24) {
                    const uint32_t row = 24u * (uint32_t)(wg - QXG_HEADS) + (uint32_t)tid;
                    if (row < 5120u) xstf(X + XO_QKV + par * XN_QKV + row, ep + 1, S.outw[tid]);
                }
                DMARK(l, 2);
            }
            // prefetch, where the workgroup waits: the router fold rows (stage O); workgroups
            // that make Q/K/V rows (idle until the context arrives) the O rows and the next
            // layer's Q/K/V rows
            load_wm(a, l, wm0, wm1);
            if (wg >= QXG_HEADS && !chunked) {
                load_o(a, l, wo, S.wo[wave_id()]);
                if (pre) load_wq(a, ln, wq, S.wq[wave_id()]);
            }
            // ---------------------------------------------------------- stage A
            if (chunked) {
                // the chunk workgroups' partial results, every workgroup's merge, then the O
                // rows and next layer's Q/K/V rows of the workgroups that make Q/K/V rows (loads
                // complete in order: issued before a poll, they would delay it)
                if ((uint32_t)wg < 4u * chunk_count(pos) && !attention_chunk_part(a, l, pos, ep + 1, S, ctl, last)) return;
                DMARK(l, 4);
                if (!attention_merge(a, l, pos, ep + 2, S, ctl, last, rec ? (int)rrow : -1)) return;
                if (wg >= QXG_HEADS) {   // (the context exchange hides them)
                    load_o(a, l, wo, S.wo[wave_id()]);
                    if (pre) load_wq(a, ln, wq, S.wq[wave_id()]);
                }
            } else if (wg < QXG_HEADS) {
                if (!attn_wait(a, l, ep + 1, S, ctl)) return;
                DMARK(l, 3);
                attention(a, l, pos, ep + 1, ap, S, last, rec ? (int)rrow : -1);
                DMARK(l, 4);
            } else {
                // While the attention runs, the other workgroups touch every translation page
                // of this layer's routed-expert rows once per XCD (workgroup w runs on XCD w % 8):
                // the expert rows picked in stage G then miss only the CU's own translation
                // cache, not the XCD's.  One 4-byte load per page, lanes on distinct pages.
                const uint32_t xi = (uint32_t)wg / 8u - 4u;   // 0 .. 27 among the XCD's non-attention workgroups
                const uint64_t gub = uni64((uint64_t)a.GU.base) + (uint64_t)l * uni64(a.GU.stride);
                const uint64_t dnb = uni64((uint64_t)a.DN.base) + (uint64_t)l * uni64(a.DN.stride);
                const uint64_t ngu = (uint64_t)a.experts * 768 * QXD_GU_UNIT, ndn = (uint64_t)a.experts * 2048 * QXD_DN_ROW;
                constexpr uint64_t PAGE = QXD_TLB_PAGE;
                const uint64_t pgu = (ngu + PAGE - 1) / PAGE, pdn = (ndn + PAGE - 1) / PAGE;
                const int tid = tix();
                if (tid < 64) {
                    uint32_t acc = 0u;
                    for (uint64_t pg = xi + 28u * (uint64_t)tid; pg < pgu + pdn; pg += 28u * 64u) {
                        const uint64_t ad = pg < pgu ? gub + pg * PAGE : dnb + (pg - pgu) * PAGE;
                        acc ^= __builtin_nontemporal_load((const GLB uint32_t *)ad);
                    }
                    if (acc == 0x9e3779b9u && tid == 64) S.flag[0] = acc;   // keeps the loads (never true: tid < 64)
                }
            }
            // ---------------------------------------------------------- stage O
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                // sentinels: words 128 h and 128 h + 64 (the two store instructions of head h)
                if constexpr (CHUNKED) QXD_SLEEP(QXD_SLEEP_CX);
                if (!wait_xch2<4>(X + XO_CX + par * XN_CX, 4096, ep + 2, S.u.m.vin, Ident(), S, ctl))
                    return;
                DMARK(l, 5);
                wait_loads();   // the O rows in LDS
                load_w8(plane(a, PL_FFN_NORM, l), fnw);   // for stage G
                const float *cx = reinterpret_cast<const float *>(S.u.m.vin);
                double b_part = 0.0;
                if ((uint32_t)wg < E) {   // router ctx-part: sum_j M[e,j] ctx_j over values 8 tid ..
                    const float4 c0 = reinterpret_cast<const float4 *>(cx)[2 * tid], c1 = reinterpret_cast<const float4 *>(cx)[2 * tid + 1];
                    double cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                    if constexpr (Q8) {
                        // the O projection sees the context as Q8_K blocks (d * code), and the
                        // fold M = W diag(w) O must see what it sees: the codes of chunk tid,
                        // as vec_digits forms them below (whole waves: wg < E is uniform)
                        const float c8[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                        uint32_t h0, h1;
                        const double dq = q8_chunk(c8, h0, h1);
#pragma unroll
                        for (int i = 0; i < 8; ++i) cv[i] = dq * (double)(int8_t)(((i < 4 ? h0 : h1) >> (8 * (i & 3))) & 255u);
                    }
                    b_part = (double)wm0.x * cv[0] + (double)wm0.y * cv[1] + (double)wm0.z * cv[2] + (double)wm0.w * cv[3] +
                             (double)wm1.x * cv[4] + (double)wm1.y * cv[5] + (double)wm1.z * cv[6] + (double)wm1.w * cv[7];
                    b_part = wave_total_d(b_part);
                    if (lane == 0) S.red[wave] = b_part;
                    __syncthreads();   // (uniform: wg < E)
                    if (tid < 2) {   // the logit before the 1/rms(x') factor, (hi, lo) words
                        double bsum = ((S.red[0] + S.red[1]) + (S.red[2] + S.red[3])) + ((S.red[4] + S.red[5]) + (S.red[6] + S.red[7]));
                        // a non-finite context makes every O output 0 (below, the reference's
                        // non-finite rule), so x' = x and the context adds nothing to the logit
                        if (!isfinite(bsum)) bsum = 0.0;
                        const uint64_t bits = (uint64_t)__double_as_longlong(a_part + bsum);
                        xst(X + XO_LG + par * XN_LG + 2 * wg + tid, ep + 3, tid == 0 ? (uint32_t)(bits >> 32) : (uint32_t)bits);
                    }
                }
                const bool ok = vec_digits<4096, false, Q8>(cx, nullptr, S);   // ends with barriers
                if (Q8 && !ok && tid == 0) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_INPUT;
                DMARK(l, 14);
                Dig g0, g1;
                load_dig(S.dig, lane, g0);
                load_dig(S.dig, lane + 64, g1);
                float part[1], out[1];
                {
                    const uint4(*lo)[64] = S.wo[wave_id()];
                    part[0] = dot_iq4<Q8, true>(lo[0][lane], wo.m0, ib, g0) + dot_iq4<Q8, true>(lo[1][lane], wo.m1, ib, g1);
                }
                rows_reduce<1>(part, out, lane);
                const int r = 8 * wg + wave;
                const float o = (ok && isfinite(out[0])) ? out[0] : 0.0f;
                if (lane == 0) {
                    S.outw[wave] = S.xs[r] + o;
                    S.oatt[wave] = o;   // (dumped in stage D, after the x publish)
                }
                __syncthreads();
                if (tid < 8) xstf(X + XO_XP + par * XN_XP + 8 * wg + tid, ep + 3, S.outw[tid]);
                DMARK(l, 6);
            }
            // ---------------------------------------------------------- stage G
            uint32_t ids[QXG_TOPK];
            {
                const int tid = tix(), lane = tid & 63, wave = tid >> 6, ib = lane & 7;
                const int gw = NWV * wg + wave;
                // The E router logits first (hi and lo words; the router workgroups publish them in
                // stage O before x', so they are normally in by now).  Then the halves work in
                // parallel: waves 0..3 (one per SIMD) take the top-8, issue the routed experts' row
                // copies for themselves and waves 4..7 and wait for them; waves 4..7 poll x' and
                // form its normalised digits.  One barrier joins them before the dots.
                const uint32_t *lgw = S.lgw;
                auto logit = [&](uint32_t e) {
                    return __longlong_as_double((long long)(((uint64_t)lgw[2 * e] << 32) | lgw[2 * e + 1]));
                };
                const int wv = wave_id();
                if (wv < 4) {
                    // the logits, polled by these four waves alone (threads 0 .. 127, a pair
                    // each), so waves 4..7 poll x' meanwhile; a failed poll is seen after the
                    // barrier below
                    if (!poll_pairs<1, 256, 0>(X + XO_LG + par * XN_LG, 2 * (int)E, ep + 3, S.lgw, Ident(), ctl)) S.fail = 1u;
                    lower_waves_sync(S, ep + 3);
                    DMARK(l, 7);
                    const double l0 = lane < (int)E ? logit(lane) : 0.0, l1 = lane + 64 < (int)E ? logit(lane + 64) : 0.0;
                    wave_top8_ids(l0, l1, (int)E, ids);
#pragma unroll
                    for (int q = 0; q < QXG_TOPK; ++q) ids[q] = ids[q] < E ? ids[q] : 0u;
                    DMARK(l, 16);
                    if (wv == 0 && lane < QXG_TOPK) {   // the picks for every wave's down rows (stage D)
                        uint32_t e = 0u;
#pragma unroll
                        for (int q = 0; q < QXG_TOPK; ++q)
                            if (q == lane) e = ids[q];
                        S.dne[lane] = e;
                    }
                    const uint64_t gub = uni64((uint64_t)a.GU.base) + (uint64_t)l * uni64(a.GU.stride);
                    uint64_t ga[7];
                    uint32_t go[7];
                    addr_gu_wg(ids, wv, gub, ga, go);
                    DMARK(l, 35);
                    u32x4 g[7];
                    load_rows(ga, g);
                    DMARK(l, 8);
#pragma unroll
                    for (int i = 0; i < 7; ++i)   // (the barrier below publishes them)
                        *reinterpret_cast<u32x4 *>(S.u.m.gu[0] + go[i]) = g[i];
                    DMARK(l, 19);
                } else {
                    // x', polled by these four waves alone (waves 0..3 are issuing the expert
                    // rows meanwhile; a poll behind those loads would wait for them)
                    const GLB uint64_t *xpb = X + XO_XP + par * XN_XP;
                    QXD_SLEEP(QXD_SLEEP_XP);
                    if (!poll_pairs<4, 256, 256>(xpb, 2048, ep + 3, reinterpret_cast<uint32_t *>(S.xp), Ident(), ctl))
                        S.fail = 1u;
                    DMARKT(l, 38, 256);
                    // RMSNorm of x' (reference src/qx_format.c:3358-3371, a double sum of squares):
                    // each thread over the 8 values it polled (pairs t + 256 k), then its wave;
                    // the four waves' sums are added after the sync below, in the same order in
                    // every workgroup
                    {
                        const int t = tid - 256;
                        double s8 = 0.0;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float2 v = *reinterpret_cast<const float2 *>(S.xp + 2 * (t + 256 * k));
                            s8 += (double)v.x * (double)v.x;
                            s8 += (double)v.y * (double)v.y;
                        }
                        s8 = wave_total_d(s8);
                        if (lane == 0) S.ssp[wv - 4] = s8;
                    }
                    upper_waves_sync(S, ep + 3);
                    DMARKT(l, 9, 256);
                    // ... and the digits of values 512 (w - 4) ..
                    const double ss = (S.ssp[0] + S.ssp[1]) + (S.ssp[2] + S.ssp[3]);
                    const double inv = 1.0 / sqrt(ss / 2048.0 + 1.0e-6);
                    DMARKT(l, 37, 256);
                    if (wv == 4 && lane == 0) S.xinv = inv;
                    const int c = 64 * (wv - 4) + lane;   // chunk of 8 values; fnw holds their weights
                    float y[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) y[k] = (float)((double)S.xp[8 * c + k] * inv) * fnw[k];
                    if constexpr (Q8) {   // (waves 4..7 whole; a non-finite x' fails the step)
                        bool fq = true;
#pragma unroll
                        for (int k = 0; k < 8; ++k) fq = fq && isfinite(y[k]);
                        if (__ballot(!fq) != 0 && lane == 0) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_INPUT;
                        store_q8(y, c, S.dig);
                    } else {
                        float mx = 0.0f;
#pragma unroll
                        for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(y[k]));   // h of a non-finite row is 0 by itself
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
                    DMARKT(l, 17, 256);
                }
                __syncthreads();
                if (S.fail) return;   // (read by every thread after the barrier: uniform)
                DMARK(l, 20);
                if (wg == 0 && wv == 0) {   // renormalised weights of the picks (reference :5265-5290)
                    const double inv = S.xinv;
                    const double l0 = lane < (int)E ? logit(lane) : 0.0, l1 = lane + 64 < (int)E ? logit(lane + 64) : 0.0;
                    double wts[QXG_TOPK];
                    uint32_t pk[QXG_TOPK];   // the picks again, from LDS (the registers of ids are free after the row loads)
#pragma unroll
                    for (int q = 0; q < QXG_TOPK; ++q) pk[q] = S.dne[q];
                    wave_top8_weights<true>(l0 * inv, l1 * inv, pk, wts);
                    if (lane < 2 * QXG_TOPK) {   // lane 2q: hi word of weight q, lane 2q + 1: lo word
                        double wl = 0.0;
                        uint32_t il = 0u;
#pragma unroll
                        for (int q = 0; q < QXG_TOPK; ++q) if ((lane >> 1) == q) { wl = wts[q]; il = pk[q]; }
                        const uint64_t bits = (uint64_t)__double_as_longlong(wl);
                        xst(X + XO_WT + par * XN_WT + lane, ep + 4, (lane & 1) ? (uint32_t)bits : (uint32_t)(bits >> 32));
                        if (rec && a.d_rids && !(lane & 1)) { gpw(a.d_rids)[8 * rrow + (lane >> 1)] = il; gpw(a.d_rw)[8 * rrow + (lane >> 1)] = wl; }
                    }
                }
                Dig g;
                load_dig(S.dig, lane, g);
                float p[8], o[8];
                {
                    // waves 0..3 take 4 of the workgroup's 24 units, waves 4..7 two (the older
                    // wave of a SIMD issues first: with 3 each, waves 4..7 finished 1 us later)
                    const uint32_t b = lane >> 3, ib = lane & 7;
                    const uint32_t q = b * 64 + ib * 8, sc = b * 8 + ib, d = b * 2;
                    const uint8_t *ub = S.u.m.gu[0] + (wv < 4 ? 4 * wv : 16 + 2 * (wv - 4)) * QXD_GU_UNIT;
                    if (wv < 4) gu_dots<4, Q8>(ub, q, sc, d, S, g, p);
                    else gu_dots<2, Q8>(ub, q, sc, d, S, g, p);
                }
                rows_reduce<8>(p, o, lane);
                DMARK(l, 18);
                DMARKT(l, 28, 256);
                DMARKT(l, 30, 448);
                (void)ib;
                (void)gw;
                {   // lane k < units: unit k (selects, then one pass for the lanes)
                    float gv = o[0], uv = o[4];
#pragma unroll
                    for (int k = 1; k < 4; ++k)
                        if (lane == k) { gv = o[k]; uv = o[4 + k]; }
                    // q8_k_compat fails the step on a non-finite expert row (src/qx_format.c:4771)
                    if (Q8 && lane < (wave < 4 ? 4 : 2) && (!isfinite(gv) || !isfinite(uv))) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_EXPERT;
                    gv = isfinite(gv) ? gv : 0.0f;
                    uv = isfinite(uv) ? uv : 0.0f;
                    if (lane < (wave < 4 ? 4 : 2)) {
                        // reference src/qx_format.c:5298, 2511-2513: h = silu(g) * u, here in f32
                        // (relative error ~1e-7 against the reference's double)
                        const float sg = gv / (1.0f + expf(-gv));
                        S.outw[(wave < 4 ? 4 * wave : 16 + 2 * (wave - 4)) + lane] = sg * uv;
                    }
                }
                __syncthreads();
                DMARK(l, 29);
                if (tid < 24) xstf(X + XO_H + par * XN_H + 24 * wg + tid, ep + 4, S.outw[tid]);
                DMARK(l, 31);
                // each wave's down rows (rank w), copied to LDS behind the gate/up dots: the h
                // poll waits behind these copies, which arrive within the exchange
                dma_dn(a, l, S.dne[wave_id()], E, S.u.m.dn[wave_id()]);
                DMARK(l, 10);
            }
            // ---------------------------------------------------------- stage D
            {
                const int tid = tix(), lane = tid & 63;
                // h and the 8 expert weights (hi, lo words)
                QXD_SLEEP(QXD_SLEEP_H);
                if (!wait_xch2<7>(X, 6144 + 16, ep + 4, S.u.m.vin,
                                   [par](int i) { return i < 6144 ? (int)(XO_H + par * XN_H) + i : (int)(XO_WT + par * XN_WT) + i - 6144; }, S, ctl))
                    return;
                DMARK(l, 11);
                wait_loads();   // the down rows (copied before the poll's loads, so already in)
                if (pre) load_wr(a, ln, wo);   // the next layer's router row
                const uint32_t *wtw = S.u.m.vin + 6144;
                double wr[QXG_TOPK];
#pragma unroll
                for (int q = 0; q < QXG_TOPK; ++q)
                    wr[q] = __longlong_as_double((long long)(((uint64_t)wtw[2 * q] << 32) | wtw[2 * q + 1]));
                // wave w: the digits of rank w's h (values 768 w .., digit groups 24 w ..), which
                // only its own dots read: no workgroup barrier (the h poll's barrier ordered
                // them after every wave's stage G reads of the digit area).  A non-finite h
                // zeroes that rank's rows only, as the reference's per-row rule does.
                const int j8 = lane >> 3, k = lane & 7, wv = wave_id();
                bool fh = true;
                {
                    const float *hv = reinterpret_cast<const float *>(S.u.m.vin) + 768 * wv;
#pragma unroll
                    for (int rd = 0; rd < 2; ++rd) {   // chunk lane, then chunk 64 + lane (lanes < 32)
                        const int c = 64 * rd + lane;
                        if (!Q8 && c >= 96) break;   // (whole quads: lanes 32.. of the second round)
                        float y[8];
                        if (c < 96) {
                            const float4 a0 = reinterpret_cast<const float4 *>(hv)[2 * c], a1 = reinterpret_cast<const float4 *>(hv)[2 * c + 1];
                            y[0] = a0.x; y[1] = a0.y; y[2] = a0.z; y[3] = a0.w; y[4] = a1.x; y[5] = a1.y; y[6] = a1.z; y[7] = a1.w;
                        } else {
#pragma unroll
                            for (int i = 0; i < 8; ++i) y[i] = 0.0f;
                        }
#pragma unroll
                        for (int i = 0; i < 8; ++i) fh = fh && isfinite(y[i]);
                        const int cg = 96 * wv + c;   // chunk of the 6144
                        if constexpr (Q8) {   // (whole wave: a 256-value block is 32 lanes)
                            uint32_t h0, h1;
                            const float dq = q8_chunk(y, h0, h1);
                            if (c < 96) {
                                uint32_t *d = S.dig + (cg >> 2) * DIG_STRIDE;
                                const int q = cg & 3;
                                *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
                                *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(0u, 0u);
                                *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(0u, 0u);
                                if (q == 0) d[24] = __float_as_uint(dq * (1.0f / 65536.0f));
                            }
                        } else {
                            float mx = 0.0f;
#pragma unroll
                            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(y[i]));
                            mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
                            mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
                            uint32_t h0, h1, m0, m1, l0, l1;
                            float sc;
                            digits8(y, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
                            uint32_t *d = S.dig + (cg >> 2) * DIG_STRIDE;
                            const int q = cg & 3;
                            *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
                            *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
                            *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
                            if (q == 0) d[24] = __float_as_uint(sc);
                        }
                    }
                }
                const bool okh = __ballot(!fh) == 0;
                if (Q8 && !okh && lane == 0) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_INPUT;
                wave_lds_sync();   // the wave's digits, read by its own lanes below
                DMARK(l, 15);
                // wave w: rank w's rows 8 wg + j (lanes 8 j .. 8 j + 7, sub-block k of each block)
                float part = 0.0f;
                {
                    // the three blocks' index words first, then block b + 1's codebook reads
                    // and digits in flight while block b computes
                    const uint8_t *dn = S.u.m.dn[wv] + j8 * QXD_DN_ROW;
                    uint2 qs[3];
                    uint32_t aux[3], ds[3];
#pragma unroll
                    for (int b = 0; b < 3; ++b) {
                        qs[b] = *reinterpret_cast<const uint2 *>(dn + 64 * b + 8 * k);
                        aux[b] = *reinterpret_cast<const uint32_t *>(dn + 192 + 32 * b + 4 * k);
                        ds[b] = *reinterpret_cast<const uint16_t *>(dn + 288 + 2 * b);
                    }
                    Iq3Look kl[2];
                    Dig gd[2];
                    iq3_look(qs[0], aux[0], S.g3, S.sel, kl[0]);
                    load_dig(S.dig, 24 * wv + k, gd[0]);
#pragma unroll
                    for (int b = 0; b < 3; ++b) {
                        if (b + 1 < 3) {
                            iq3_look(qs[b + 1], aux[b + 1], S.g3, S.sel, kl[(b + 1) & 1]);
                            load_dig(S.dig, 24 * wv + 8 * (b + 1) + k, gd[(b + 1) & 1]);
                        }
                        part += iq3_dot<Q8, true>(kl[b & 1], aux[b], ds[b], gd[b & 1]);
                    }
                }
                part += dppf<DPP_XOR1>(part);
                part += dppf<DPP_XOR2>(part);
                part += dppf<DPP_HALF_MIRROR>(part);   // lanes 8 j .. 8 j + 7 hold row j's sum
                if (Q8 && okh && k == 0 && !isfinite(part)) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_EXPERT;
                if (k == 0) S.ys[wv][j8] = (okh && isfinite(part)) ? part : 0.0f;
                DMARK(l, 26);
                __syncthreads();
                DMARK(l, 27);
                if (tid < 8) {
                    // reference src/qx_format.c:5296-5309: moe += (float)(w_r * (double)y_r), rank order
                    float moe = 0.0f;
#pragma unroll
                    for (int q = 0; q < QXG_TOPK; ++q) moe += (float)(wr[q] * (double)S.ys[q][tid]);
                    const int r = 8 * wg + tid;
                    const float xn = S.xp[r] + moe;
                    xstf(X + XO_X + ((l + 1) & 1) * XN_X + r, ep + 5, xn);
                    if (rec) {   // the recorded step's dumps, after the publish (off the layer's critical path)
                        if (a.d_layer) gpw(a.d_layer)[rrow * 2048 + r] = xn;
                        if (a.d_half) {
                            gpw(a.d_half)[rrow * 4096 + r] = S.oatt[tid];
                            gpw(a.d_half)[rrow * 4096 + 2048 + r] = moe;
                        }
                        if (a.d_res && l + 1 == L) gpw(a.d_res)[rslot * 2048 + r] = xn;
                    }
                }
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
            if (!wait_xch2<2>(X + XO_X + (L & 1) * XN_X, 2048, eph, reinterpret_cast<uint32_t *>(S.xs), Ident(), S, ctl))
                return;
            DMARK(48, 1);
            if (tid == 0) S.u.hd.next = 0u;   // (published by the barrier in vec_digits)
            const bool fin = vec_digits<2048, true, Q8>(S.xs, onw, S, nullptr, rec && a.d_norm ? gpw(a.d_norm) + rslot * 2048 : nullptr);
            if (Q8 && !fin && tid == 0) gpw(a.st)->q8_fault = QXG_Q8_NONFINITE_INPUT;   // (src/qx_format.c:4026-4027)
            float bv;
            uint32_t bi;
            bool nonfin;
            DMARK(48, 2);
            head_rows<Q8>(a, S, fin, bv, bi, nonfin, rslot);
            DMARK(48, 3);
            DMARKT(48, 6, 64);
            DMARKT(48, 7, 192);
            DMARKT(48, 8, 256);
            DMARKT(48, 9, 448);
            if (nonfin) gpw(a.st)->nonfinite = 1u;
            // workgroup best, then every workgroup reads all the bests
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const uint32_t oi = __shfl_xor(bi, o);
                if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            if (lane == 0) { S.u.hd.bv[wave] = bv; S.u.hd.bi[wave] = bi; }
            __syncthreads();
            DMARK(48, 5);
            if (tid < 2) {
                float v = S.u.hd.bv[0];
                uint32_t i = S.u.hd.bi[0];
                for (int w = 1; w < NWV; ++w)
                    if (better(S.u.hd.bv[w], S.u.hd.bi[w], v, i)) { v = S.u.hd.bv[w]; i = S.u.hd.bi[w]; }
                xst(X + XO_AM + (step & 1) * XN_AM + 2 * wg + tid, eph + 1, tid == 0 ? __float_as_uint(v) : i);
            }
            if (!wait_xch2<1>(X + XO_AM + (step & 1) * XN_AM, XN_AM, eph + 1, S.u.hd.am, Ident(), S, ctl))
                return;
            DMARK(48, 4);
            // layer 0's rows for the next step, after the argmax exchange: issued earlier, its
            // poll would wait behind them (loads complete in order); none after the last step
            if (!last) {
                if (wg >= QXG_HEADS) load_wq(a, 0, wq, S.wq[wave_id()]);
                load_wr(a, 0, wo);
            }
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
    wait_loads();   // no copy into LDS outstanding at exit (a launch of no steps has the prologue's)
    if (a.d_time && wg == 0 && tix() == 0) gpw(a.d_time)[a.rec_base + a.steps] = __builtin_amdgcn_s_memrealtime();
#ifdef QXD_TRACE
    __syncthreads();
    if (threadIdx.x < 5 * 40) {
        const int sl = threadIdx.x / 40, pt = threadIdx.x % 40;
        qxd_trace_buf[sl < 4 ? 20 + sl : 48][pt][blockIdx.x] = qxd_tl[sl][pt];
    }
#endif
}

extern "C" __global__ __launch_bounds__(NT, 1) void qxk_decode(QxDArgs args) { decode_steps<false, false>(args); }
extern "C" __global__ __launch_bounds__(NT, 1) void qxk_decode_chunked(QxDArgs args) { decode_steps<true, false>(args); }
// the same in the q8_k_compat activation mode (every matvec input as Q8_K blocks)
extern "C" __global__ __launch_bounds__(NT, 1) void qxk_decode_q8(QxDArgs args) { decode_steps<false, true>(args); }
extern "C" __global__ __launch_bounds__(NT, 1) void qxk_decode_chunked_q8(QxDArgs args) { decode_steps<true, true>(args); }

// The routed experts' rows of one layer in the interleaved layout (QXD_GU_UNIT, QXD_DN_ROW),
// from the IQ2_XS gate/up planes (qs 64, sc 8, d 2 bytes per block, 8 blocks per row) and
// the IQ3_XXS down planes (qs 64, aux 32, d 2 per block, 3 blocks per row): one thread per
// gate/up unit or down row.  The block scales d are stored saturated (fp16_sat), so the
// decode's dots convert them with the plain hardware conversion.
extern "C" __global__ __launch_bounds__(256) void qxk_interleave_experts(const uint8_t *gq, const uint8_t *gs, const uint8_t *gd,
                                                                          const uint8_t *uq, const uint8_t *us, const uint8_t *ud,
                                                                          const uint8_t *dq, const uint8_t *dx, const uint8_t *dd,
                                                                          uint32_t E, uint8_t *gu, uint8_t *dn) {
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x, ngu = (uint64_t)E * 768, ndn = (uint64_t)E * 2048;
    auto cp32 = [](uint8_t *dst, const uint8_t *src, int words) {
        for (int i = 0; i < words; ++i) reinterpret_cast<uint32_t *>(dst)[i] = reinterpret_cast<const uint32_t *>(src)[i];
    };
    auto cp_d16 = [](uint8_t *dst, const uint8_t *src, int n) {   // block scales, saturated
        for (int i = 0; i < n; ++i)
            reinterpret_cast<uint16_t *>(dst)[i] = (uint16_t)fp16_sat(reinterpret_cast<const uint16_t *>(src)[i]);
    };
    if (t < ngu) {
        uint8_t *o = gu + t * QXD_GU_UNIT;
        cp32(o, gq + t * 512, 128);
        cp32(o + 512, gs + t * 64, 16);
        cp_d16(o + 576, gd + t * 16, 8);
        cp32(o + 592, uq + t * 512, 128);
        cp32(o + 1104, us + t * 64, 16);
        cp_d16(o + 1168, ud + t * 16, 8);
    } else if (t < ngu + ndn) {
        const uint64_t r = t - ngu, e = r / 2048, row = r % 2048;   // source: row-major per expert
        uint8_t *o = dn + (((row >> 3) * E + e) * 8 + (row & 7)) * QXD_DN_ROW;
        cp32(o, dq + r * 192, 48);
        cp32(o + 192, dx + r * 96, 24);
        uint16_t *o16 = reinterpret_cast<uint16_t *>(o + 288);
        const uint16_t *d16 = reinterpret_cast<const uint16_t *>(dd + r * 6);
        for (int i = 0; i < 8; ++i) o16[i] = i < 3 ? (uint16_t)fp16_sat(d16[i]) : (uint16_t)0;
    }
}

// A given row through the KV quantizer (int8_mag, int8_scale, int8_code): one workgroup of 256
// threads, n <= 4096 values (the same-input seam of qxg_int8_quantize).
extern "C" __global__ __launch_bounds__(256) void qxk_int8_row(const float *x, uint32_t n, int8_t *codes, float *scale) {
    __shared__ float red[4];
    float mx = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, int8_mag(x[i]));
    mx = wave_max_f(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float sc = int8_scale(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    for (uint32_t i = threadIdx.x; i < n; i += 256) codes[i] = int8_code(x[i], sc);
    if (threadIdx.x == 0) *scale = sc;
}

// The Q6_K head rows in the interleaved layout (QXD_HEAD_ROW): one thread per row, from the
// ql (128), qh (64), sc (16) and d (2) planes of its 8 blocks.
extern "C" __global__ __launch_bounds__(256) void qxk_interleave_head(const uint8_t *ql, const uint8_t *qh, const uint8_t *sc,
                                                                       const uint8_t *d, uint32_t vocab, uint8_t *out) {
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= vocab) return;
    auto cp32 = [](uint8_t *dst, const uint8_t *src, int words) {
        for (int i = 0; i < words; ++i) reinterpret_cast<uint32_t *>(dst)[i] = reinterpret_cast<const uint32_t *>(src)[i];
    };
    uint8_t *o = out + r * QXD_HEAD_ROW;
    cp32(o, ql + r * 1024, 256);
    cp32(o + 1024, qh + r * 512, 128);
    cp32(o + 1536, sc + r * 128, 32);
    cp32(o + 1664, d + r * 16, 4);
}

// The decode packs of one layer (QXD_PK_*): workgroup w of the grid (256) copies pack w:
// for w >= 32 its 24 Q/K/V row slots (stacked rows [Q 4096 | K 512 | V 512] 24 (w - 32) ..,
// zero past row 5119) with their 8-byte block metas; for every w its O rows 8 w .. 8 w + 7
// and metas; for w < experts the router row and router-fold row of expert w.  The metas'
// scale halves are stored saturated (fp16_sat), as are the expert layouts' below.
extern "C" __global__ __launch_bounds__(256) void qxk_pack_decode(const uint8_t *qq, const uint8_t *qm, const uint8_t *kq,
                                                                   const uint8_t *km, const uint8_t *vq, const uint8_t *vm,
                                                                   const uint8_t *oq, const uint8_t *om, const float *router,
                                                                   const float *mfold, uint32_t experts, uint8_t *out) {
    const uint32_t w = blockIdx.x;
    uint8_t *o = out + (uint64_t)w * QXD_PK_BYTES;
    auto cp = [](uint8_t *dst, const uint8_t *src, uint32_t bytes) {
        for (uint32_t i = threadIdx.x; i < bytes / 16; i += 256)
            reinterpret_cast<uint4 *>(dst)[i] = reinterpret_cast<const uint4 *>(src)[i];
    };
    // two IQ4_XS block metas {d | scales_h << 16, scales_l}, their scale halves saturated
    auto sat_meta = [](uint4 m) {
        m.x = (m.x & 0xffff0000u) | fp16_sat(m.x & 0xffffu);
        m.z = (m.z & 0xffff0000u) | fp16_sat(m.z & 0xffffu);
        return m;
    };
    // one Q/K/V row slot: 1024 qs bytes (64 chunks) or 64 meta bytes (4 chunks) of row `row`
    auto slot = [&](uint32_t s, bool meta) -> const uint4 * {
        const uint32_t row = 24u * (w - QXG_HEADS) + s;
        if (row >= 5120u) return nullptr;
        const uint32_t rb = meta ? 64u : 1024u;
        const uint8_t *p = row < 4096u ? (meta ? qm : qq) + (uint64_t)row * rb
                         : row < 4608u ? (meta ? km : kq) + (uint64_t)(row - 4096u) * rb
                                       : (meta ? vm : vq) + (uint64_t)(row - 4608u) * rb;
        return reinterpret_cast<const uint4 *>(p);
    };
    if (w >= QXG_HEADS) {
        for (uint32_t i = threadIdx.x; i < 24u * 64u; i += 256) {
            const uint4 *src = slot(i / 64u, false);
            reinterpret_cast<uint4 *>(o + QXD_PK_QQ)[i] = src ? src[i % 64u] : make_uint4(0u, 0u, 0u, 0u);
        }
        for (uint32_t i = threadIdx.x; i < 24u * 4u; i += 256) {
            const uint4 *src = slot(i / 4u, true);
            reinterpret_cast<uint4 *>(o + QXD_PK_QM)[i] = src ? sat_meta(src[i % 4u]) : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    cp(o + QXD_PK_OQ, oq + (uint64_t)w * 8 * 2048, 16384);
    for (uint32_t i = threadIdx.x; i < 1024u / 16u; i += 256)
        reinterpret_cast<uint4 *>(o + QXD_PK_OM)[i] = sat_meta(reinterpret_cast<const uint4 *>(om + (uint64_t)w * 8 * 128)[i]);
    if (w < experts) {   // (workgroups past the experts read pack experts - 1's)
        cp(o + QXD_PK_RT, reinterpret_cast<const uint8_t *>(router + (uint64_t)w * 2048), 8192);
        cp(o + QXD_PK_MF, reinterpret_cast<const uint8_t *>(mfold + (uint64_t)w * 4096), 16384);
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
