// Persistent decode kernel: every layer of one token in one launch on gfx950.
//
// Grid: QXG_PBLOCKS workgroups of 256 threads, one per CU (the LDS footprint
// admits one workgroup per CU).  Each layer runs as six phases (reference
// src/qx_format.c:6282-6423 for attention, 5198-5317 for the MoE):
//   P1 attn RMSNorm + Q/K/V IQ4_XS rows      (all waves, 5 rows each)
//   P2 q/k norm, RoPE, INT8 KV append, GQA   (workgroups 0..31, one q head each)
//   P3 O projection + residual                (all waves, 2 rows each)
//   P4 ffn RMSNorm + digits, router logits    (all; waves of workgroups 0..31 own one expert)
//   P5 top-8, gate/up IQ2_XS + SwiGLU         (all waves, 6 units each)
//   P6 down IQ3_XXS, weighted sum + residual  (all waves, the same 2 rows as P3)
// A phase hands its output to the next through "tagged" 64-bit words
// {epoch:32, f32 bits:32}, written and read with relaxed agent-scope atomics
// (single-copy atomic, coherent across XCDs without cache maintenance).  A
// consumer polls until every word it needs carries the current epoch, so no
// barrier, counter or fence is needed; a wait is bounded by a deadline and a
// shared abort flag, so every wave exits even if a producer never arrives.
// Every exchange buffer has two slots (layer parity): a slot is rewritten two
// layers later, after a chain of all-to-all dependencies that every reader of
// the old contents has passed.
//
// Loads return in issue order, so a poll issued behind outstanding weight loads
// cannot complete before them.  Every weight load is therefore issued right after
// a poll has completed, one phase ahead of its use: the O rows and the attention's
// cached K/V rows after P1's input arrives, the router rows after P3's, the next
// layer's Q/K/V rows after P6's; only the routed experts' rows wait for the top-8.
#include "qxg_dev.h"

#ifdef QXG_TRACE
__device__ unsigned long long qxg_ptrace_buf[96][16][4 * QXG_PBLOCKS];
extern "C" int qxg_ptrace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(qxg_ptrace_buf), sizeof(qxg_ptrace_buf)) == hipSuccess;
}
// phase timestamps for development builds only: lane 0 of each wave stores
// s_memrealtime (100 MHz) into qxg_ptrace_buf[sub-layer][point][wave]
#define PMARK(sub, p)                                                                       \
    do {                                                                                    \
        const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();                     \
        if ((threadIdx.x & 63) == 0 && (sub) < 96)                                         \
            qxg_ptrace_buf[sub][p][blockIdx.x * 4 + (threadIdx.x >> 6)] = t_;               \
    } while (0)
#else
#define PMARK(sub, p) ((void)0)
#endif

namespace {

#define GLB __attribute__((address_space(1)))

// Wave-uniform values.  The compiler's divergence analysis neither knows that
// threadIdx.x / 64 is the same in every lane of a wave nor that a pointer read from
// LDS is; readfirstlane puts such values in scalar registers, so the per-wave
// arithmetic and branches are scalar and the pointers address global memory (not flat).
DEV uint64_t uni64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
template <typename T>
DEV const GLB T *gptr(const T *p) { return (const GLB T *)uni64((uint64_t)p); }
template <typename T>
DEV GLB T *gptrw(T *p) { return (GLB T *)uni64((uint64_t)p); }
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
DEV uint4 gld4(const GLB void *p) { const u32x4 v = *(const GLB u32x4 *)p; return make_uint4(v.x, v.y, v.z, v.w); }
DEV uint2 gld2(const GLB void *p) { const u32x2 v = *(const GLB u32x2 *)p; return make_uint2(v.x, v.y); }

DEV uint64_t ld_tag(const GLB uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void st_bits(GLB uint64_t *p, uint32_t bits, uint32_t ep) {
    __hip_atomic_store(p, ((uint64_t)ep << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void st_tag(GLB uint64_t *p, float v, uint32_t ep) { st_bits(p, __float_as_uint(v), ep); }

struct Ctl {
    uint64_t deadline;
    uint32_t *abort;
};

// true while the wait may go on; every 64 polls checks the deadline and the abort flag
DEV bool keep_waiting(uint32_t &it, const Ctl &c) {
    if ((++it & 63u) != 0) return true;
    if (wall_clock64() > c.deadline ||
        __hip_atomic_load(c.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
        __hip_atomic_store(c.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return true;
}

// Waits until every p[idx[k]] carries epoch ep; the f32 payloads go to v.  All loads
// are issued before the first check; later rounds reload only the stale words.
template <int K>
DEV bool wait_tagged(const GLB uint64_t *p, const int (&idx)[K], uint32_t ep, uint32_t (&v)[K], const Ctl &c) {
    uint64_t w[K];
#pragma unroll
    for (int k = 0; k < K; ++k) w[k] = ld_tag(p + idx[k]);
    uint32_t it = 0;
    for (;;) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < K; ++k) all = all && (uint32_t)(w[k] >> 32) == ep;
        if (all) break;
        if (!keep_waiting(it, c)) return false;
#pragma unroll
        for (int k = 0; k < K; ++k)
            if ((uint32_t)(w[k] >> 32) != ep) w[k] = ld_tag(p + idx[k]);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = (uint32_t)w[k];
    return true;
}

// LDS address-space view of a __shared__ location (the direct-to-LDS loads take one)
typedef __attribute__((address_space(3))) void lds_void;
DEV lds_void *lds_ptr(void *p) { return (lds_void *)p; }
constexpr int CPOL_SC1 = 16;   // agent-scope coherent access (bypasses the non-coherent L2 copy)

// Wave-level wait for the chunks (128 tagged words = 1 KiB each) wave, wave+4, ... of a
// tagged vector, loaded straight into the LDS stage (raw {f32 bits, epoch} pairs) with
// agent-coherent direct-to-LDS loads: lane i fetches words 2i, 2i+1 of a chunk.  Stale
// chunks are fetched again until every word carries the epoch.  false on timeout/abort.
DEV bool wave_poll_chunks(const GLB uint64_t *src, uint32_t ep, uint2 *stage, int nchunks, const Ctl &c) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int mine = (nchunks - wave + 3) >> 2;
    uint32_t pending = mine >= 32 ? 0xffffffffu : (1u << mine) - 1u, it = 0;
    for (;;) {
        for (uint32_t m = pending; m; m &= m - 1) {
            const int ch = wave + 4 * __builtin_ctz(m);
            __builtin_amdgcn_global_load_lds((const GLB void *)(src + 128 * ch + 2 * lane), lds_ptr(stage + 128 * ch), 16, 0, CPOL_SC1);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the LDS copies have landed
        uint32_t stale = 0;
        for (uint32_t m = pending; m; m &= m - 1) {
            const int k = __builtin_ctz(m), ch = wave + 4 * k;
            const uint4 v = *reinterpret_cast<const uint4 *>(stage + 128 * ch + 2 * lane);
            if (__ballot(v.y != ep || v.w != ep)) stale |= 1u << k;
        }
        pending = stale;
        if (!pending) return true;
        if (!keep_waiting(it, c)) return false;
    }
}

// the stage from a plain f32 vector (the residual entering the launch's first sub-layer)
DEV void stage_plain(const GLB float *x, int n, uint2 *stage) {
    for (int i = threadIdx.x; i < n; i += 256) stage[i] = make_uint2(__float_as_uint(x[i]), 0u);
}

// 8 consecutive staged values [8c, 8c+8)
DEV void stage8(const uint2 *stage, int c, float (&v)[8]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(stage + 8 * c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 t = p[k];
        v[2 * k] = __uint_as_float(t.x);
        v[2 * k + 1] = __uint_as_float(t.z);
    }
}

DEV void digits_store(const float (&v)[8], float mx, int c, uint32_t *s_dig) {
    uint32_t h0, h1, m0, m1, l0, l1;
    float sc;
    digits8(v, isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
    uint32_t *d = s_dig + (c >> 2) * DIG_STRIDE;
    const int q = c & 3;
    *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
    *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
    *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
    if (q == 0) d[24] = __float_as_uint(sc);
}

// Digit planes (groups of 32 = 4 threads x 8 values) of the staged vector of 8*nch
// values into s_dig.  With w8 (the thread's 8 norm weights; nch == 256) the vector is
// first RMS-normalised (reference src/qx_format.c:3358-3371; xn written to norm_out
// when given).  Returns true when every value is finite; ends with a block barrier.
DEV bool digits_stage(const uint2 *stage, int nch, const float *w8, uint32_t *s_dig, double *s_red, float *norm_out) {
    const int tid = threadIdx.x;
    bool fin = true;
    if (w8) {
        float v[8];
        stage8(stage, tid, v);
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
        ss = wave_total_d(ss);
        if ((tid & 63) == 0) s_red[tid >> 6] = ss;
        __syncthreads();
        const double tot = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
        const double inv = 1.0 / sqrt(tot / 2048.0 + 1.0e-6);
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = (float)((double)v[i] * inv) * w8[i];
            fin = fin && isfinite(v[i]);
            mx = fmaxf(mx, fabsf(v[i]));
        }
        if (norm_out) {
            reinterpret_cast<float4 *>(norm_out)[2 * tid] = make_float4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<float4 *>(norm_out)[2 * tid + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
        digits_store(v, mx, tid, s_dig);
    } else {
#pragma unroll 1
        for (int c = tid; c < nch; c += 256) {
            float v[8];
            stage8(stage, c, v);
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) { fin = fin && isfinite(v[i]); mx = fmaxf(mx, fabsf(v[i])); }
            mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
            mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
            digits_store(v, mx, c, s_dig);
        }
    }
    return __syncthreads_or(!fin) == 0;
}

// Router top-8 by one wave (reference src/qx_format.c:5265-5285; the order and tie
// rules are those of wave_top8): lane q < 8 ends with pick q's expert id and its
// renormalised weight e_q / sum_r e_r, e = exp(l - l_max).  Rounds are a rolled loop.
DEV void top8_lanes(double l0, double l1, int E, uint32_t &my_id, double &my_w) {
    const int lane = threadIdx.x & 63;
    my_id = 0;
    bool tie = false;
    {
        uint32_t k0 = lane < E ? fkey(l0) : 0u, k1 = lane + 64 < E ? fkey(l1) : 0u;
#pragma unroll 1
        for (int r = 0; r < QXG_TOPK; ++r) {
            const uint32_t m = wave_max_u32(max(k0, k1));
            const uint64_t b0 = __ballot(m != 0u && k0 == m), b1 = __ballot(m != 0u && k1 == m);
            tie = tie || (__popcll(b0) + __popcll(b1) > 1);
            const uint32_t id = b0 ? (uint32_t)__builtin_ctzll(b0) : b1 ? 64u + (uint32_t)__builtin_ctzll(b1) : 0u;
            if (lane == r) my_id = id;
            if (lane == (int)(id & 63u)) { if (id < 64u) k0 = 0u; else k1 = 0u; }
        }
    }
    if (tie) {   // several experts at a maximal f32 key: redo with the exact keys of the doubles
        uint64_t k0 = lane < E ? dkey(l0) : 0ull, k1 = lane + 64 < E ? dkey(l1) : 0ull;
#pragma unroll 1
        for (int r = 0; r < QXG_TOPK; ++r) {
            const uint64_t m = wave_max_u64(umax64(k0, k1));
            const uint64_t b0 = __ballot(m != 0ull && k0 == m), b1 = __ballot(m != 0ull && k1 == m);
            const uint32_t id = b0 ? (uint32_t)__builtin_ctzll(b0) : b1 ? 64u + (uint32_t)__builtin_ctzll(b1) : 0u;
            if (lane == r) my_id = id;
            if (lane == (int)(id & 63u)) { if (id < 64u) k0 = 0ull; else k1 = 0ull; }
        }
    }
    const double a0 = __shfl(l0, (int)(my_id & 63u)), a1 = __shfl(l1, (int)(my_id & 63u));
    const double lq = my_id < 64u ? a0 : a1;
    const double lmax = rdlaned(lq, 0);
    const double eq = lane < QXG_TOPK ? exp(lq - lmax) : 0.0;
    double sel = 0.0;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) sel += rdlaned(eq, q);   // rank order, as the reference
    my_w = eq / sel;
}

// layer l's plane `id` (scalar arithmetic on the arguments)
template <typename T>
DEV const GLB T *plane(const QxPArgs &a, int id, uint32_t l) {
    return (const GLB T *)(uni64((uint64_t)a.P[id].base) + (uint64_t)l * uni64(a.P[id].stride));
}

DEV void load8(const GLB float *p, float (&w)[8]) {
    const f32x4 a = ((const GLB f32x4 *)p)[0], b = ((const GLB f32x4 *)p)[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}
DEV void load32g(const GLB float *p, float *v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 t = ((const GLB f32x4 *)p)[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

constexpr int ATT_STAGE = 128;   // cached KV positions staged in LDS by the attention workgroups

struct AttnLds {
    double sc[QXG_MAX_CTX];
    uint4 kst[ATT_STAGE * 8], vst[ATT_STAGE * 8];
    float kss[ATT_STAGE], vss[ATT_STAGE];
    float k[512], v[512];
    double q[128];
    double redd[4];
    float red[4];
    float part[2][128];
    int8_t k8[128], v8[128];
    float scale[2];
};

struct Lds {
    uint4 g2[512];
    uint2 g3[256];
    uint2 sel[128];
    uint32_t dig[192 * DIG_STRIDE];
    double red[4];
    float xn[2048];      // normalised ffn input (router waves)
    uint32_t lg[256];    // router logits as (hi, lo) words
    union {
        AttnLds att;                        // P2 (attention workgroups)
        uint2 stage[QXG_TOPK * QXG_FFN];    // polled tagged input vectors of P1, P3, P4, P6
    };
};

// ---------------------------------------------------------------- P2 attention
// One q head per workgroup (reference qx_rope_gqa_attention_partial,
// src/qx_format.c:5051-5196): per-head q/k RMSNorm (3740-3757), RoPE from the
// host table (4625-4641), INT8 K/V quantization of the current position over all
// 512 values (4449-4463; workgroup 0 stores the row, every workgroup derives the
// same row), double scores and softmax, f32 context accumulated per position in
// position order within two halves of the positions.
struct AttnPre {   // loaded in P1, after its input has arrived
    uint4 kst[4], vst[4];
    float kss, vss, kw0, kw1, qw0, qw1;
    double cs, sn;
};

DEV void attn_prefetch(const QxPArgs &a, uint32_t l, uint32_t pos, AttnPre &p) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int kvh = blockIdx.x >> 3;
    const uint64_t base = (uint64_t)l * a.ctx;
    const uint32_t nst = pos < (uint32_t)ATT_STAGE ? pos : (uint32_t)ATT_STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        if (t < nst) {
            const uint64_t off = (base + t) * 512 + kvh * 128 + 16 * (tid & 7);
            p.kst[i] = gld4(gptr(a.kc) + off);
            p.vst[i] = gld4(gptr(a.vc) + off);
        }
    }
    p.kss = (uint32_t)tid < nst ? gptr(a.ks)[base + tid] : 0.0f;
    p.vss = (uint32_t)tid < nst ? gptr(a.vs)[base + tid] : 0.0f;
    const GLB float *kn = plane<float>(a, PL_K_NORM, l), *qn = plane<float>(a, PL_Q_NORM, l);
    p.kw0 = kn[lane]; p.kw1 = kn[64 + lane];
    p.qw0 = qn[lane]; p.qw1 = qn[64 + lane];
    p.cs = gptr(a.T.rope_cos)[pos * 64 + lane];
    p.sn = gptr(a.T.rope_sin)[pos * 64 + lane];
}

DEV bool attn_phase(const QxPArgs &a, uint32_t l, uint32_t pos, const GLB uint64_t *qkv, GLB uint64_t *cx, uint32_t ep,
                    const AttnPre &p, AttnLds &S, const Ctl &c) {
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int qh = blockIdx.x, kvh = qh >> 3;
    const uint32_t n = pos + 1;
    const uint64_t base = (uint64_t)l * a.ctx;
    const uint32_t nst = pos < (uint32_t)ATT_STAGE ? pos : (uint32_t)ATT_STAGE;
    const int idx[6] = {4096 + 128 * wave + lane, 4096 + 128 * wave + 64 + lane, 4608 + tid, 4608 + 256 + tid,
                        128 * qh + lane, 128 * qh + 64 + lane};
    uint32_t in[6];
    const bool got = wait_tagged<6>(qkv, idx, ep, in, c);
    if (__syncthreads_or(!got)) return false;
    PMARK(2 * l, 4);
    float k0 = __uint_as_float(in[0]), k1 = __uint_as_float(in[1]);
    const float v0 = __uint_as_float(in[2]), v1 = __uint_as_float(in[3]);
    float q0 = __uint_as_float(in[4]), q1 = __uint_as_float(in[5]);
    head_norm_rope_wave(k0, k1, p.kw0, p.kw1, p.cs, p.sn);
    S.k[128 * wave + lane] = k0;
    S.k[128 * wave + 64 + lane] = k1;
    S.v[tid] = v0;
    S.v[256 + tid] = v1;
    if (wave == 0) {
        head_norm_rope_wave(q0, q1, p.qw0, p.qw1, p.cs, p.sn);
        S.q[lane] = (double)q0;
        S.q[64 + lane] = (double)q1;
    }
    float ka, va;
    {
        const float a0 = isfinite(k0) ? fabsf(k0) : 0.0f, a1 = isfinite(k1) ? fabsf(k1) : 0.0f;
        ka = fmaxf(a0, a1);
        const float b0 = isfinite(v0) ? fabsf(v0) : 0.0f, b1 = isfinite(v1) ? fabsf(v1) : 0.0f;
        va = fmaxf(b0, b1);
    }
    ka = block_max256(ka, S.red);
    va = block_max256(va, S.red);
    const float kscale = ka > 0.0f ? ka / 127.0f : 1.0f, vscale = va > 0.0f ? va / 127.0f : 1.0f;
    const uint64_t slot = base + pos;
    for (int i = tid; i < 512; i += 256) {
        const float kx = S.k[i], vx = S.v[i];
        int qk = isfinite(kx) ? (int)rintf(kx / kscale) : 0;
        int qv = isfinite(vx) ? (int)rintf(vx / vscale) : 0;
        qk = qk < -127 ? -127 : qk > 127 ? 127 : qk;
        qv = qv < -127 ? -127 : qv > 127 ? 127 : qv;
        if (blockIdx.x == 0) { gptrw(a.kc)[slot * 512 + i] = (int8_t)qk; gptrw(a.vc)[slot * 512 + i] = (int8_t)qv; }
        if ((i >> 7) == kvh) { S.k8[i & 127] = (int8_t)qk; S.v8[i & 127] = (int8_t)qv; }
    }
    if (blockIdx.x == 0 && tid == 0) { gptrw(a.ks)[slot] = kscale; gptrw(a.vs)[slot] = vscale; }
    if (blockIdx.x == 0 && a.d_vcur) { gptrw(a.d_vcur)[tid] = v0; gptrw(a.d_vcur)[256 + tid] = v1; }
    if (tid == 0) { S.scale[0] = kscale; S.scale[1] = vscale; }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        if (t < nst) { S.kst[t * 8 + (tid & 7)] = p.kst[i]; S.vst[t * 8 + (tid & 7)] = p.vst[i]; }
    }
    if ((uint32_t)tid < nst) { S.kss[tid] = p.kss; S.vss[tid] = p.vss; }
    __syncthreads();
    PMARK(2 * l, 12);
    {   // scores: 16 lanes per position, 8 dims per lane
        const int sub = lane >> 4, dl = lane & 15;
        double qd[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qd[j] = S.q[8 * dl + j];
        for (uint32_t t0 = 4 * wave; t0 < n; t0 += 16) {
            const uint32_t t = t0 + sub;
            double acc = 0.0;
            if (t < n) {
                uint2 kk;
                float ksc;
                if (t == pos) {
                    kk = *reinterpret_cast<const uint2 *>(S.k8 + 8 * dl);
                    ksc = S.scale[0];
                } else if (t < nst) {
                    kk = reinterpret_cast<const uint2 *>(S.kst)[t * 16 + dl];
                    ksc = S.kss[t];
                } else {
                    kk = gld2(gptr(a.kc) + (base + t) * 512 + kvh * 128 + 8 * dl);
                    ksc = gptr(a.ks)[base + t];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int8_t kb = (int8_t)(((j < 4 ? kk.x : kk.y) >> (8 * (j & 3))) & 255u);
                    acc += qd[j] * (double)((float)kb * ksc);
                }
            }
            acc = row16_sum_d(acc);
            if (t < n && dl == 0) {
                double sc = acc / a.sqrt_hd;
                if (!isfinite(sc)) sc = 0.0;
                S.sc[t] = sc;
            }
        }
    }
    __syncthreads();
    PMARK(2 * l, 13);
    double mx = -1.0e300;
    for (uint32_t t = tid; t < n; t += 256) mx = fmax(mx, S.sc[t]);
    mx = wave_max_d(mx);
    if (lane == 0) S.redd[wave] = mx;
    __syncthreads();
    mx = fmax(fmax(S.redd[0], S.redd[1]), fmax(S.redd[2], S.redd[3]));
    double den = 0.0;
    for (uint32_t t = tid; t < n; t += 256) {
        const double e = exp(S.sc[t] - mx);
        S.sc[t] = e;
        den += e;
    }
    den = wave_total_d(den);
    __syncthreads();
    if (lane == 0) S.redd[wave] = den;
    __syncthreads();
    den = (S.redd[0] + S.redd[1]) + (S.redd[2] + S.redd[3]);
    if (!isfinite(den) || den <= 0.0) den = 1.0;
    PMARK(2 * l, 14);
    const int d = tid & 127, hf = tid >> 7;
    const uint32_t t0 = hf ? n / 2 : 0, t1 = hf ? n : n / 2;
    float acc = 0.0f;
    for (uint32_t t = t0; t < t1; ++t) {
        const double wgt = S.sc[t] / den;
        const float vv = t == pos ? (float)S.v8[d] * S.scale[1]
                         : t < nst ? (float)reinterpret_cast<const int8_t *>(S.vst)[t * 128 + d] * S.vss[t]
                                   : (float)gptr(a.vc)[(base + t) * 512 + kvh * 128 + d] * gptr(a.vs)[base + t];
        acc += (float)(wgt * (double)vv);
    }
    S.part[hf][d] = acc;
    __syncthreads();
    if (tid < 128) {
        const float o = S.part[0][tid] + S.part[1][tid];
        st_tag(cx + qh * 128 + tid, o, ep);
        if (a.d_ctx) gptrw(a.d_ctx)[qh * 128 + tid] = o;
    }
    __syncthreads();   // the LDS area is reused as the next phase's stage
    return true;
}

// P1 weights of one wave: Q/K/V rows 5gw .. 5gw+4 (lane = 8*block + sub-block)
struct P1W {
    uint4 q[5];
    uint2 m[5];
};
DEV void load_p1(const QxPArgs &a, uint32_t l, int gw, int lane, P1W &w) {
    const int b = lane >> 3, ib = lane & 7;
#pragma unroll
    for (int rr = 0; rr < 5; ++rr) {
        const int r = 5 * gw + rr;
        const GLB uint8_t *qs, *meta;
        int lr;
        if (r < 4096) { qs = plane<uint8_t>(a, PL_Q_QS, l); meta = plane<uint8_t>(a, PL_Q_META, l); lr = r; }
        else if (r < 4608) { qs = plane<uint8_t>(a, PL_K_QS, l); meta = plane<uint8_t>(a, PL_K_META, l); lr = r - 4096; }
        else { qs = plane<uint8_t>(a, PL_V_QS, l); meta = plane<uint8_t>(a, PL_V_META, l); lr = r - 4608; }
        const uint64_t blk = (uint64_t)lr * 8 + b;
        w.q[rr] = gld4(qs + blk * 128 + 16 * ib);
        w.m[rr] = gld2(meta + blk * 8);
    }
}
// P3 weights of one wave: O rows 2gw, 2gw+1 (16 blocks per row; lane takes blocks lane/8 and 8+lane/8)
struct P3W {
    uint4 q0[2], q1[2];
    uint2 m0[2], m1[2];
};
DEV void load_p3(const QxPArgs &a, uint32_t l, int gw, int lane, P3W &w) {
    const int ib = lane & 7, b0 = lane >> 3, b1 = 8 + (lane >> 3);
    const GLB uint8_t *oq = plane<uint8_t>(a, PL_O_QS, l), *om = plane<uint8_t>(a, PL_O_META, l);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const uint64_t k0 = (uint64_t)(2 * gw + rr) * 16 + b0, k1 = (uint64_t)(2 * gw + rr) * 16 + b1;
        w.q0[rr] = gld4(oq + k0 * 128 + 16 * ib);
        w.q1[rr] = gld4(oq + k1 * 128 + 16 * ib);
        w.m0[rr] = gld2(om + k0 * 8);
        w.m1[rr] = gld2(om + k1 * 8);
    }
}

}  // namespace

// ================================================================= kernel
extern "C" __global__ __launch_bounds__(256, 1) void qxk_layers(QxPArgs args) {
    __shared__ Lds S;
    // The arguments are copied to LDS and read from there where used: reads of LDS
    // cannot be hoisted across the phase barriers, so the ~40 pointers are not held in
    // scalar registers for the whole launch.
    __shared__ QxPArgs a;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    static_assert(sizeof(QxPArgs) % 8 == 0 && sizeof(QxPArgs) <= 256 * 8, "argument copy");
    if (tid < (int)(sizeof(QxPArgs) / 8))
        reinterpret_cast<uint64_t *>(&a)[tid] = reinterpret_cast<const uint64_t *>(&args)[tid];
    __syncthreads();
    const int gw = blockIdx.x * 4 + wave;   // global wave, 0 .. 4*QXG_PBLOCKS-1
    const int ib = lane & 7;
    const Ctl ctl{wall_clock64() + a.timeout, a.abort};
    const uint32_t l0 = a.s0 >> 1, l1 = (a.s1 + 1) >> 1;   // layers touched by [s0, s1)
    // Q/K/V rows and attn-norm weights of the next attention half, fetched one phase ahead
    P1W w1;
    float anw[8];
    if ((a.s0 & 1) == 0 && a.s0 < a.s1) {
        load_p1(a, l0, gw, lane, w1);
        load8(plane<float>(a, PL_ATTN_NORM, l0) + 8 * tid, anw);
    }
    S.g2[tid] = gld4(gptr(a.T.g2) + tid);
    S.g2[tid + 256] = gld4(gptr(a.T.g2) + tid + 256);
    S.g3[tid] = gld2(gptr(a.T.g3) + tid);
    if (tid < 128) S.sel[tid] = gld2(gptr(a.T.sel) + tid);
    const GLB DevState *st = gptr(a.st_w);
    const uint32_t pos = __builtin_amdgcn_readfirstlane(st->pos0 + st->step);
    const uint32_t ep_base = __builtin_amdgcn_readfirstlane(st->epoch);
    // residual rows 2gw, 2gw+1 live in this wave (wave-uniform) for the whole launch
    float xo0 = gptr(a.x_in)[2 * gw], xo1 = gptr(a.x_in)[2 * gw + 1];
    const int E = (int)a.experts;
    __syncthreads();
#pragma unroll 1
    for (uint32_t l = l0; l < l1; ++l) {
        const uint32_t slot = l & 1, sa = 2 * l, sm = 2 * l + 1;
        const bool run_a = sa >= a.s0 && sa < a.s1, run_m = sm >= a.s0 && sm < a.s1;
        const uint32_t epa = ep_base + (sa - a.s0) + 1, epm = ep_base + (sm - a.s0) + 1;
        // router rows of P4 (workgroups 0..31: one expert per wave) and ffn-norm weights
        const bool router = blockIdx.x < 32 && (uint32_t)gw < a.experts && run_m;
        float rw[32], fnw[8];
        if (run_a) {
            // ------------------------------------------------ P1: RMSNorm + Q/K/V rows
            GLB uint64_t *qkv = gptrw(a.qkv) + slot * 5120;
            PMARK(sa, 0);
            P3W w3;
            AttnPre ap;
            {
                bool got = true;
                if (sa == a.s0) stage_plain(gptr(a.x_in), 2048, S.stage);
                else got = wave_poll_chunks(gptr(a.xb) + ((l + 1) & 1) * 2048, epa - 1, S.stage, 16, ctl);
                if (__syncthreads_or(!got)) return;
                PMARK(sa, 1);
                load_p3(a, l, gw, lane, w3);
                if (blockIdx.x < QXG_HEADS) attn_prefetch(a, l, pos, ap);
                const bool ok = digits_stage(S.stage, 256, anw, S.dig, S.red, nullptr);
                PMARK(sa, 2);
                Dig g;
                load_dig(S.dig, lane, g);
                // rows in a rolled loop: the prefetch registers and the results shift by
                // one slot per iteration, so every index is static
                float part[8], out[8];
#pragma unroll 1
                for (int rr = 0; rr < 5; ++rr) {
                    const float d = dot_iq4(w1.q[0], w1.m[0], ib, g);
#pragma unroll
                    for (int k = 0; k + 1 < 5; ++k) { w1.q[k] = w1.q[k + 1]; w1.m[k] = w1.m[k + 1]; part[k] = part[k + 1]; }
                    part[4] = d;
                }
                part[5] = part[6] = part[7] = 0.0f;
                rows_reduce<8>(part, out, lane);
                float mine = 0.0f;
#pragma unroll
                for (int rr = 0; rr < 5; ++rr) if (lane == rr) mine = out[rr];
                if (lane < 5) st_tag(qkv + 5 * gw + lane, (ok && isfinite(mine)) ? mine : 0.0f, epa);
                PMARK(sa, 3);
            }
            // ------------------------------------------------ P2: attention (q head per workgroup)
            GLB uint64_t *cx = gptrw(a.cx) + slot * 4096;
            if (blockIdx.x < QXG_HEADS) {
                if (!attn_phase(a, l, pos, qkv, cx, epa, ap, S.att, ctl)) return;
                PMARK(sa, 5);
            }
            // ------------------------------------------------ P3: O projection + residual
            {
                const bool got = wave_poll_chunks(cx, epa, S.stage, 32, ctl);
                if (__syncthreads_or(!got)) return;
                PMARK(sa, 6);
                if (router) load32g(plane<float>(a, PL_ROUTER, l) + (uint64_t)gw * 2048 + 32 * lane, rw);
                load8(plane<float>(a, PL_FFN_NORM, l) + 8 * tid, fnw);
                const bool ok = digits_stage(S.stage, 512, nullptr, S.dig, S.red, nullptr);
                PMARK(sa, 7);
                Dig g0, g1;
                load_dig(S.dig, lane, g0);
                load_dig(S.dig, lane + 64, g1);
                float part[2], out[2];
#pragma unroll 1
                for (int rr = 0; rr < 2; ++rr) {
                    const float d = dot_iq4(w3.q0[0], w3.m0[0], ib, g0) + dot_iq4(w3.q1[0], w3.m1[0], ib, g1);
                    w3.q0[0] = w3.q0[1]; w3.m0[0] = w3.m0[1]; w3.q1[0] = w3.q1[1]; w3.m1[0] = w3.m1[1];
                    part[0] = part[1];
                    part[1] = d;
                }
                rows_reduce<2>(part, out, lane);
                GLB uint64_t *xa = gptrw(a.xa) + slot * 2048;
                const float o0 = (ok && isfinite(out[0])) ? out[0] : 0.0f, o1 = (ok && isfinite(out[1])) ? out[1] : 0.0f;
                xo0 = xo0 + o0;
                xo1 = xo1 + o1;
                if (lane < 2) {
                    st_tag(xa + 2 * gw + lane, lane ? xo1 : xo0, epa);
                    if (a.d_attn) gptrw(a.d_attn)[2 * gw + lane] = lane ? o1 : o0;
                }
                PMARK(sa, 8);
            }
        }
        if (run_m) {
            // ------------------------------------------------ P4: ffn RMSNorm + digits, router logits
            PMARK(sm, 0);
            if (!run_a) {
                if (router) load32g(plane<float>(a, PL_ROUTER, l) + (uint64_t)gw * 2048 + 32 * lane, rw);
                load8(plane<float>(a, PL_FFN_NORM, l) + 8 * tid, fnw);
            }
            bool got = true;
            if (sm == a.s0) stage_plain(gptr(a.x_in), 2048, S.stage);
            else got = wave_poll_chunks(gptr(a.xa) + slot * 2048, epm - 1, S.stage, 16, ctl);
            if (__syncthreads_or(!got)) return;
            PMARK(sm, 1);
            // digits of the normalised input (for P5); xn kept in LDS for the router waves
            const bool ok = digits_stage(S.stage, 256, fnw, S.dig, S.red, S.xn);
            PMARK(sm, 2);
            GLB uint64_t *lg = gptrw(a.lg) + slot * 256;
            if (router) {
                // reference src/qx_format.c:5254-5264: logit_e = sum_i double(W[e,i]) * double(xn_i)
                double acc = 0.0;
#pragma unroll
                for (int i = 0; i < 32; ++i) acc += (double)rw[i] * (double)S.xn[32 * lane + i];
                acc = wave_total_d(acc);
                if (lane == 0) {
                    const uint64_t bits = (uint64_t)__double_as_longlong(acc);
                    st_bits(lg + 2 * gw, (uint32_t)(bits >> 32), epm);
                    st_bits(lg + 2 * gw + 1, (uint32_t)bits, epm);
                }
                PMARK(sm, 3);
            }
            // ------------------------------------------------ P5: top-8, gate/up + SwiGLU
            GLB uint64_t *hb = gptrw(a.hb) + slot * (QXG_TOPK * QXG_FFN);
            {   // one wave polls the 2E logit words (fewer pollers on a few hot lines)
                bool got2 = true;
                if (wave == 0) {
                    int idx[4];
                    uint32_t v[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) idx[k] = lane + 64 * k < 2 * E ? lane + 64 * k : 0;
                    got2 = wait_tagged<4>(lg, idx, epm, v, ctl);
#pragma unroll
                    for (int k = 0; k < 4; ++k) S.lg[lane + 64 * k] = v[k];
                }
                if (__syncthreads_or(!got2)) return;
            }
            PMARK(sm, 4);
            auto logit = [&](int ex) {
                return __longlong_as_double((long long)(((uint64_t)S.lg[2 * ex] << 32) | S.lg[2 * ex + 1]));
            };
            uint32_t my_id;
            double my_w;
            top8_lanes(lane < E ? logit(lane) : 0.0, lane + 64 < E ? logit(lane + 64) : 0.0, E, my_id, my_w);
            my_id = my_id < a.experts ? my_id : 0u;
            PMARK(sm, 10);
            const int b = lane >> 3;
            const int u0 = 6 * gw;                    // 768 = 128 * 6: one expert per wave
            const uint32_t ue = (uint32_t)__builtin_amdgcn_readlane((int)my_id, u0 / QXG_FFN);
            const GLB uint8_t *g_qs = plane<uint8_t>(a, PL_G_QS, l), *g_sc = plane<uint8_t>(a, PL_G_SC, l);
            const GLB uint8_t *u_qs = plane<uint8_t>(a, PL_U_QS, l), *u_sc = plane<uint8_t>(a, PL_U_SC, l);
            const GLB uint16_t *g_d = plane<uint16_t>(a, PL_G_D, l), *u_d = plane<uint16_t>(a, PL_U_D, l);
            uint2 gq[6], uq[6];
            uint32_t gs[6], us[6], gd[6], ud[6];
#pragma unroll
            for (int uu = 0; uu < 6; ++uu) {
                const int i = (u0 + uu) % QXG_FFN;
                const uint64_t blk = ((uint64_t)ue * QXG_FFN + i) * 8 + b;
                gq[uu] = gld2(g_qs + blk * 64 + 8 * ib);
                uq[uu] = gld2(u_qs + blk * 64 + 8 * ib);
                gs[uu] = g_sc[blk * 8 + ib];
                us[uu] = u_sc[blk * 8 + ib];
                gd[uu] = g_d[blk];
                ud[uu] = u_d[blk];
            }
            // down weights of P6 (rows 2gw, 2gw+1): lanes 8r..8r+7 hold rank r, lane 8r+k sub-block k of 3 blocks
            const int dr = lane >> 3, dk = lane & 7;
            const uint32_t de = (uint32_t)__shfl((int)my_id, dr);
            const GLB uint8_t *d_qs = plane<uint8_t>(a, PL_D_QS, l), *d_aux = plane<uint8_t>(a, PL_D_AUX, l);
            const GLB uint16_t *d_d = plane<uint16_t>(a, PL_D_D, l);
            uint2 dq[6];
            uint32_t dax[6], ddv[6];
#pragma unroll
            for (int t = 0; t < 6; ++t) {   // t = 3*row + block
                const uint64_t blk = ((uint64_t)de * 2048 + 2 * gw + t / 3) * 3 + t % 3;
                dq[t] = gld2(d_qs + blk * 64 + 8 * dk);
                dax[t] = *(const GLB uint32_t *)(d_aux + blk * 32 + 4 * dk);
                ddv[t] = d_d[blk];
            }
            if (blockIdx.x == 0 && wave == 0 && lane < QXG_TOPK) {   // ids and weights for the MoE replay seam
                gptrw(a.st_w)->moe_ids[lane] = my_id;
                gptrw(a.st_w)->moe_w[lane] = my_w;
            }
            PMARK(sm, 5);
            {
                Dig g;
                load_dig(S.dig, lane, g);
                // unit by unit in a rolled loop: the prefetch registers and the results
                // shift by one slot per iteration, so every index stays static and the
                // codebook reads of one unit are in flight at a time
                float pg[6], pu[6];
#pragma unroll 1
                for (int uu = 0; uu < 6; ++uu) {
                    const float ag = dot_iq2(gq[0], gs[0], gd[0], g, S.g2, S.sel);
                    const float au = dot_iq2(uq[0], us[0], ud[0], g, S.g2, S.sel);
#pragma unroll
                    for (int k = 0; k + 1 < 6; ++k) {
                        gq[k] = gq[k + 1]; uq[k] = uq[k + 1]; gs[k] = gs[k + 1]; us[k] = us[k + 1];
                        gd[k] = gd[k + 1]; ud[k] = ud[k + 1]; pg[k] = pg[k + 1]; pu[k] = pu[k + 1];
                    }
                    pg[5] = ag;
                    pu[5] = au;
                }
                float p[16], o[16];
#pragma unroll
                for (int k = 0; k < 8; ++k) { p[k] = k < 6 ? pg[k < 6 ? k : 0] : 0.0f; p[8 + k] = k < 6 ? pu[k < 6 ? k : 0] : 0.0f; }
                rows_reduce<16>(p, o, lane);
                float gv = 0.0f, uv = 0.0f;
#pragma unroll
                for (int k = 0; k < 6; ++k) if (lane == k) { gv = o[k]; uv = o[8 + k]; }
                if (lane < 6) {
                    gv = (ok && isfinite(gv)) ? gv : 0.0f;
                    uv = (ok && isfinite(uv)) ? uv : 0.0f;
                    // reference src/qx_format.c:5298, 2511-2513: h = (float)(silu((double)g) * (double)u)
                    const double sg = (double)gv / (1.0 + exp(-(double)gv));
                    st_tag(hb + u0 + lane, (float)(sg * (double)uv), epm);
                }
                PMARK(sm, 6);
            }
            // ------------------------------------------------ P6: down, weighted sum + residual
            {
                const bool got3 = wave_poll_chunks(hb, epm, S.stage, 48, ctl);
                if (__syncthreads_or(!got3)) return;
                PMARK(sm, 7);
                if (l + 1 < l1 && 2 * (l + 1) < a.s1) {   // the next layer's attention half runs
                    load_p1(a, l + 1, gw, lane, w1);
                    load8(plane<float>(a, PL_ATTN_NORM, l + 1) + 8 * tid, anw);
                }
                const bool okh = digits_stage(S.stage, 768, nullptr, S.dig, S.red, nullptr);
                PMARK(sm, 8);
                GLB uint64_t *xb = gptrw(a.xb) + slot * 2048;
#pragma unroll 1
                for (int rr = 0; rr < 2; ++rr) {
                    float part = 0.0f;
#pragma unroll 1
                    for (int j = 0; j < 3; ++j) {
                        Dig g;
                        load_dig(S.dig, 24 * dr + 8 * j + dk, g);
                        part += dot_iq3(dq[0], dax[0], ddv[0], g, S.g3, S.sel);
#pragma unroll
                        for (int k = 0; k + 1 < 6; ++k) { dq[k] = dq[k + 1]; dax[k] = dax[k + 1]; ddv[k] = ddv[k + 1]; }
                    }
                    part += dppf<DPP_XOR1>(part);
                    part += dppf<DPP_XOR2>(part);
                    part += dppf<DPP_HALF_MIRROR>(part);   // lanes 8q..8q+7 hold rank q's row
                    const float y = (okh && isfinite(part)) ? part : 0.0f;
                    // reference src/qx_format.c:5296-5309: moe += (float)(w_r * (double)y_r), rank order
                    float moe = 0.0f;
#pragma unroll
                    for (int q = 0; q < QXG_TOPK; ++q) moe += (float)(rdlaned(my_w, q) * (double)rdlanef(y, 8 * q));
                    const float xn = (rr ? xo1 : xo0) + moe;
                    if (rr) xo1 = xn; else xo0 = xn;
                    if (lane == 0) {
                        st_tag(xb + 2 * gw + rr, xn, epm);
                        if (a.d_moe) gptrw(a.d_moe)[2 * gw + rr] = moe;
                        if (a.d_layer) gptrw(a.d_layer)[(uint64_t)l * 2048 + 2 * gw + rr] = xn;
                    }
                }
                PMARK(sm, 9);
            }
        }
    }
    if (lane < 2) gptrw(a.x_out)[2 * gw + lane] = lane ? xo1 : xo0;
    // the epoch advances once every workgroup has read it (any workgroup finishing
    // implies all have passed their first phase)
    if (blockIdx.x == 0 && tid == 0) gptrw(a.st_w)->epoch = ep_base + (a.s1 - a.s0) + 1;
}
