// CDNA4 (gfx950) kernels for one-token Qwen3-30B-A3B decode.
//
// Built with -ffp-contract=off: every multiply-add below is either a separate
// rounded multiply and add (where the reference's op order must be kept) or an
// explicit fmaf.
//
// Dequant-matvec scheme.  Every weight of the formats used here is, exactly,
//     w = (per-block f32 scale) * (small integer code)
// (IQ2_XS d*(2s+1)/8 * grid*sign, IQ3_XXS d*(2a+1)/4 * grid*sign,
//  IQ4_XS d*(ls-32) * kvalue, Q6_K d*sc * (q-32)); the f32 products the reference
// forms (src/qx_format.c:1914-2169 of the reference) are exact, so
//     sum_i w_i x_i = scale * sum_i code_i x_i
// holds in exact arithmetic.  Each activation group of 32 values is written as
// x_i = s * (H_i*2^16 + M_i*2^8 + L_i) with s a power of two and signed int8
// digits (22 significant bits, |error| <= 2^-23 * max|x_group|), so the inner
// products are exact int32 v_dot4 sums; only the per-sub-block combination is
// rounded (f32).  Codes are formed in registers with v_perm byte lookups from
// LDS codebooks, so the kernels stream the quantized bytes once from HBM.
#include "qxg_dev.h"

#ifdef QXG_TRACE
__device__ unsigned long long qxg_trace_buf[8][8192][8];
extern "C" int qxg_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(qxg_trace_buf), sizeof(qxg_trace_buf)) == hipSuccess;
}
extern "C" int qxg_trace_clear() {
    static unsigned long long zero[8 * 8192 * 8];
    return hipMemcpyToSymbol(HIP_SYMBOL(qxg_trace_buf), zero, sizeof(zero)) == hipSuccess;
}
#endif

// ================================================================= kernels

// Q4_K embedding row of tokens[step] -> x (reference src/qx_format.c:2079-2110,
// 3759-3793).  256 threads, thread (b, l) produces 8 values of block b.
extern "C" __global__ __launch_bounds__(256) void qxk_embed(const uint8_t *emb, uint64_t row_bytes,
                                                            const uint32_t *tokens, const DevState *st, float *x) {
    embed_q4k_row(emb + (uint64_t)tokens[st->step] * row_bytes, x);
}

// attn RMSNorm + Q/K/V projections (2048 -> 4096 | 512 | 512) into qkv[5120]; each of
// the three matrices IQ4_XS or Q5_K (the real checkpoint's attn_v).  Wave per RPW
// consecutive rows; lane = 8*block + sub-block.  A workgroup's 4*RPW rows lie in one
// matrix, so its format is uniform.  Every global load of the wave is issued before the
// norm/digit prologue so their latencies overlap.
struct QkvW {
    const uint8_t *qs[3], *p1[3], *p2[3];
    uint32_t type[3];
};

template <int RPW, int FMT, bool Q8>
DEV void qkv_rows(const float *x, const float *norm_w, const uint8_t *qs, const uint8_t *p1, const uint8_t *p2, int lr0,
                  int r0, uint32_t *s_dig, double *s_red, float *qkv, DevState *st) {
    const int lane = threadIdx.x & 63;
    const int b = lane >> 3, ib = lane & 7;
    // the activation loads come first (used first) and inside the format branch, so no
    // norm arithmetic is hoisted above the branch, where it would wait for x before the
    // weight loads are issued
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    uint4 qv[RPW], qw[RPW], ha[RPW], hb[RPW], mv[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const uint64_t blk = (uint64_t)(lr0 + rr) * 8 + b;
        if constexpr (FMT == 23) {
            qv[rr] = ldw4(qs + blk * 128 + 16 * ib);
            const uint2 m = ldw2(p1 + blk * 8);
            mv[rr] = make_uint4(m.x, m.y, 0u, 0u);
        } else {
            qv[rr] = ldw4(qs + blk * 128 + 32 * (ib >> 1));
            qw[rr] = ldw4(qs + blk * 128 + 32 * (ib >> 1) + 16);
            ha[rr] = ldw4(p2 + blk * 32);
            hb[rr] = ldw4(p2 + blk * 32 + 16);
            mv[rr] = ldw4(p1 + blk * 16);
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_ANCHOR(din.v[0][7]);
    QXG_MARK(3, 1);
    const bool ok = block_act<Q8>(din, s_dig, s_red);
    QXG_MARK(3, 2);
    Dig g;
    load_dig(s_dig, lane, g);
    float part[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        if constexpr (FMT == 23) part[rr] = dot_iq4(qv[rr], make_uint2(mv[rr].x, mv[rr].y), ib, g);
        else part[rr] = dot_q5(qv[rr], qw[rr], ha[rr], hb[rr], mv[rr], ib, g);
    }
    QXG_ANCHOR(part[0]); QXG_ANCHOR(part[RPW - 1]);
    QXG_MARK(3, 3);
    float out[RPW];
    rows_reduce<RPW>(part, out, lane);
    float mine = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) if (lane == rr) mine = out[rr];
    if (lane < RPW) qkv[r0 + lane] = (ok && isfinite(mine)) ? mine : 0.0f;
    if (Q8 && !ok && threadIdx.x == 0) st->q8_fault = QXG_Q8_NONFINITE_INPUT;
    QXG_MARK(3, 4);
}

// 512 workgroups, two per CU: 0..255 take 16 Q rows each (4 per wave), 256..511 take 4 K
// or V rows each (1 per wave), so every CU holds the same 20 rows (640 workgroups of 8
// rows left half the CUs with a third workgroup).  The branch is workgroup-uniform.
template <bool Q8>
__global__ __launch_bounds__(256) void qxk_qkv(const float *x, const float *norm_w, QkvW w, float *qkv, DevState *st) {
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    const int wave = wave_id();
    QXG_MARK(3, 0);
    if (blockIdx.x < 256) {
        const int q0 = (blockIdx.x * 4 + wave) * 4;
        if (w.type[0] == 13) qkv_rows<4, 13, Q8>(x, norm_w, w.qs[0], w.p1[0], w.p2[0], q0, q0, s_dig, s_red, qkv, st);
        else qkv_rows<4, 23, Q8>(x, norm_w, w.qs[0], w.p1[0], w.p2[0], q0, q0, s_dig, s_red, qkv, st);
    } else {
        const int g0 = 4096 + ((blockIdx.x - 256) * 4 + wave);
        const int mi = g0 < 4608 ? 1 : 2, l0 = g0 - (mi == 1 ? 4096 : 4608);
        if (w.type[mi] == 13) qkv_rows<1, 13, Q8>(x, norm_w, w.qs[mi], w.p1[mi], w.p2[mi], l0, g0, s_dig, s_red, qkv, st);
        else qkv_rows<1, 23, Q8>(x, norm_w, w.qs[mi], w.p1[mi], w.p2[mi], l0, g0, s_dig, s_red, qkv, st);
    }
}

// Attention for one q head, with the per-head q/k RMSNorm (src/qx_format.c:3740-3757),
// split-half RoPE (4625-4641; cos/sin from the host-computed table) and INT8 K/V
// quantization (4449-4463) of the current position fused in: every block derives the
// same K/V row (the scale spans all 512 values), block (0, 0) stores it at
// [layer][pos], and each block uses its own copy for position pos.  Scores (a quad per
// position, q as int8 digit planes against the INT8 K codes), double softmax, f32
// context sums over 16 interleaved position groups (reference src/qx_format.c:5127-5172).
// Block (h, s) of the (32, S) grid takes positions [128 s, min(128 s + 128, pos + 1)):
// their cached K/V rows and scales are loaded at kernel start, together with q/k/v, and
// staged in LDS while the norm, RoPE and quantization run.  With one split (pos < 128)
// the block writes the normalised context; with several, each writes its unnormalised
// context sums, maximum score and exp-sum to part[h][s], and qxk_attn_merge combines
// them.  Blocks past the last split return at once; the host launches S >= (pos+128)/128.

constexpr int ATT_STAGE = QXG_ATT_SPLIT;   // positions per block (4 uint4 of K and of V per thread)

extern "C" __global__ __launch_bounds__(256) void qxk_attn(const float *qkv, const float *q_norm, const float *k_norm,
        Tables T, int8_t *kc, int8_t *vc, float *ks, float *vs, uint32_t layer, uint32_t ctx, double sqrt_hd,
        const DevState *st, float *ctx_out, float *part, float *vcur_dump, double *wsum) {
    __shared__ double s_sc[ATT_STAGE];             // scores, then weights
    __shared__ uint4 s_kst[ATT_STAGE * 8], s_vst[ATT_STAGE * 8];   // staged rows of this kv head
    __shared__ float s_kss[ATT_STAGE], s_vss[ATT_STAGE];
    __shared__ float s_k[512], s_v[512];
    __shared__ __align__(16) float s_q[128];
    __shared__ __align__(16) uint32_t s_qd[4 * DIG_STRIDE];
    __shared__ float2 red2[4];
    __shared__ double redd[8];   // score maximum [0..3], exp-sum [4..7]
    __shared__ float s_part[16][132];
    __shared__ __align__(16) int8_t s_k8[128];
    __shared__ __align__(16) int8_t s_v8[128];
    __shared__ float s_scale[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int qh = blockIdx.x, kvh = qh >> 3, split = blockIdx.y;
    QXG_MARK(4, 0);
    // the inputs that do not depend on the position first (the position is a load of its
    // own, from the device state; the RoPE row of the position is kept there as well)
    float k0 = qkv[4096 + 128 * wave + lane], k1 = qkv[4096 + 128 * wave + 64 + lane];
    const float v0 = qkv[4608 + tid], v1 = qkv[4608 + 256 + tid];
    float q0 = qkv[128 * qh + lane], q1 = qkv[128 * qh + 64 + lane];
    const float kw0 = k_norm[lane], kw1 = k_norm[64 + lane], qw0 = q_norm[lane], qw1 = q_norm[64 + lane];
    const double c = st->rope_c[lane], s = st->rope_s[lane];   // the position's row, kept in st
    // the split's cached rows: their addresses depend on the split and the cache length
    // only, so they load before the position is known (rows past the cache read the
    // split's first row, or row 0 for a split past the cache; rows the position does not
    // reach are never used).  16 bytes of row t0 + (tid>>3) + 32*i, chunk tid&7, i < 4.
    const uint32_t t0 = (uint32_t)split * ATT_STAGE;
    const uint64_t base = (uint64_t)layer * ctx;
    const uint32_t rows = t0 < ctx ? min(ctx - t0, (uint32_t)ATT_STAGE) : 0u;
    const uint32_t r0 = t0 < ctx ? t0 : 0u;
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));   // register-promoted (a uint4 array is not)
    v4u kst[4], vst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        const uint64_t off = (base + r0 + (t < rows ? t : 0u)) * 512 + kvh * 128 + 16 * (tid & 7);
        kst[i] = *reinterpret_cast<const v4u *>(kc + off);
        vst[i] = *reinterpret_cast<const v4u *>(vc + off);
    }
    const uint32_t ts = r0 + ((uint32_t)tid < rows ? (uint32_t)tid : 0u);
    const float kss = ks[base + ts], vss = vs[base + ts];
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t pos = cur_pos(st), n = pos + 1;
    const uint32_t nsplit = (n + ATT_STAGE - 1) / ATT_STAGE;
    if ((uint32_t)split >= nsplit) return;   // block-uniform
    const uint32_t cnt = min(n - t0, (uint32_t)ATT_STAGE);
    // staged (cached) positions t0 .. t0+nst-1; the last split's last position is pos
    const uint32_t nst = (uint32_t)split + 1 == nsplit ? cnt - 1 : cnt;
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_MARK(4, 1);
    head_norm_rope_wave(k0, k1, kw0, kw1, c, s);
    s_k[128 * wave + lane] = k0;
    s_k[128 * wave + 64 + lane] = k1;
    s_v[tid] = v0;
    s_v[256 + tid] = v1;
    if (wave == 0) {
        head_norm_rope_wave(q0, q1, qw0, qw1, c, s);
        s_q[lane] = q0;
        s_q[64 + lane] = q1;
    }
    // stage the split's cached rows (all 128 slots; those past nst are never read); the
    // barrier of the K/V maxima publishes them
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        reinterpret_cast<v4u *>(s_kst)[t * 8 + (tid & 7)] = kst[i];
        reinterpret_cast<v4u *>(s_vst)[t * 8 + (tid & 7)] = vst[i];
    }
    if (tid < ATT_STAGE) { s_kss[tid] = kss; s_vss[tid] = vss; }
    // INT8 quantize K and V over all 512 values (scale = max|x|/127, 1 if zero)
    float ka = fmaxf(int8_mag(k0), int8_mag(k1)), va = fmaxf(int8_mag(v0), int8_mag(v1));
    QXG_MARK(4, 2);
    block_max2_256(ka, va, red2);
    QXG_MARK(4, 3);
    const float kscale = int8_scale(ka), vscale = int8_scale(va);
    // values 2 tid and 2 tid + 1 (a 2-byte store each for K and V)
    int8_t qkb[2], qvb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = 2 * tid + j;
        qkb[j] = int8_code(s_k[i], kscale);
        qvb[j] = int8_code(s_v[i], vscale);
    }
    if ((tid >> 6) == kvh) {   // this kv head's 128 values: threads 64 kvh .. 64 kvh + 63
        reinterpret_cast<uint16_t *>(s_k8)[tid & 63] = (uint16_t)((uint8_t)qkb[0] | ((uint32_t)(uint8_t)qkb[1] << 8));
        reinterpret_cast<uint16_t *>(s_v8)[tid & 63] = (uint16_t)((uint8_t)qvb[0] | ((uint32_t)(uint8_t)qvb[1] << 8));
    }
    if (tid == 0) { s_scale[0] = kscale; s_scale[1] = vscale; }
    __syncthreads();
    QXG_MARK(4, 4);
    // local position u is t0 + u: pos from the block's own row, the others from the LDS stage
    auto krow = [&](uint32_t u, int g, uint4 (&k)[2], float &ksc) {
        if (u >= nst) {
            k[0] = reinterpret_cast<const uint4 *>(s_k8)[2 * g];
            k[1] = reinterpret_cast<const uint4 *>(s_k8)[2 * g + 1];
            ksc = s_scale[0];
        } else {
            k[0] = s_kst[u * 8 + 2 * g];
            k[1] = s_kst[u * 8 + 2 * g + 1];
            ksc = s_kss[u];
        }
    };
    auto vrow = [&](uint32_t u, int dg) -> uint2 {
        if (u >= nst) return reinterpret_cast<const uint2 *>(s_v8)[dg];
        return reinterpret_cast<const uint2 *>(s_vst)[u * 16 + dg];
    };
    auto vsc = [&](uint32_t u) -> float { return u >= nst ? s_scale[1] : s_vss[u]; };
    const double mx = attn_scores(s_q, s_qd, cnt, sqrt_hd, s_sc, redd, krow);
    QXG_MARK(4, 5);
    const bool one = nsplit == 1;
    const double den = attn_weights(cnt, mx, s_sc, redd, vsc, one, wsum ? wsum + qh : nullptr);
    QXG_MARK(4, 6);
    float *pp = part + ((uint64_t)qh * QXG_MAX_SPLITS + split) * QXG_ATT_PART;
    attn_context(cnt, s_sc, s_part, vrow, one ? ctx_out + qh * 128 : pp);
    if (!one && tid == 0) {
        reinterpret_cast<double *>(pp + 128)[0] = mx;
        reinterpret_cast<double *>(pp + 128)[1] = den;
    }
    // the current position's K/V row into the cache, last, so that no wait for these
    // stores precedes the block's own work (other splits never read slot pos)
    if (blockIdx.x == 0 && split == 0) {
        const uint64_t slot = base + pos;
        reinterpret_cast<uint16_t *>(kc + slot * 512)[tid] = (uint16_t)((uint8_t)qkb[0] | ((uint32_t)(uint8_t)qkb[1] << 8));
        reinterpret_cast<uint16_t *>(vc + slot * 512)[tid] = (uint16_t)((uint8_t)qvb[0] | ((uint32_t)(uint8_t)qvb[1] << 8));
        if (tid == 0) { ks[slot] = kscale; vs[slot] = vscale; }
        if (vcur_dump) { vcur_dump[tid] = v0; vcur_dump[256 + tid] = v1; }
    }
    QXG_MARK(4, 7);
}

// The splits of qxk_attn combined for one q head (thread = dimension): M = max_s m_s,
// w_s = exp(m_s - M), L = sum_s w_s l_s (1 if not finite and positive), ctx[d] =
// sum_s (float)(w_s / L) * acc_s[d] in split order.  With one split the attention
// kernel wrote the context itself and this returns.
// wsum (may be null): the head's sum of normalised weights, sum_s w_s l_s / L.
extern "C" __global__ __launch_bounds__(128) void qxk_attn_merge(const DevState *st, const float *part, float *ctx_out,
                                                                  double *wsum) {
    const uint32_t n = cur_pos(st) + 1, ns = (n + ATT_STAGE - 1) / ATT_STAGE;
    if (ns <= 1) return;
    const int qh = blockIdx.x, d = threadIdx.x;
    const float *p = part + (uint64_t)qh * QXG_MAX_SPLITS * QXG_ATT_PART;
    double M = -INFINITY;
    for (uint32_t s = 0; s < ns; ++s) M = fmax(M, reinterpret_cast<const double *>(p + s * QXG_ATT_PART + 128)[0]);
    double L = 0.0;
    for (uint32_t s = 0; s < ns; ++s) {
        const double *ml = reinterpret_cast<const double *>(p + s * QXG_ATT_PART + 128);
        L += exp(ml[0] - M) * ml[1];
    }
    if (!isfinite(L) || L <= 0.0) L = 1.0;
    if (wsum && d == 0) {
        double t = 0.0;
        for (uint32_t s = 0; s < ns; ++s) {
            const double *ml = reinterpret_cast<const double *>(p + s * QXG_ATT_PART + 128);
            t += exp(ml[0] - M) * ml[1] / L;
        }
        wsum[qh] = t;
    }
    float o = 0.0f;
    for (uint32_t s = 0; s < ns; ++s) {
        const double m = reinterpret_cast<const double *>(p + s * QXG_ATT_PART + 128)[0];
        o = fmaf((float)(exp(m - M) / L), p[s * QXG_ATT_PART + d], o);
    }
    ctx_out[qh * 128 + d] = o;
}

// O projection 4096 -> 2048 on ctx (IQ4_XS, or Q5_K in the real checkpoint), then
// x[r] += o[r] (src/qx_format.c:6420-6423).  Lane handles sub-blocks lane and lane+64
// (blocks lane/8 and 8+lane/8).
template <int RPW, int FMT, bool Q8>
__global__ __launch_bounds__(256) void qxk_oproj(const float *ctxv, const uint8_t *qs, const uint8_t *meta,
                                                  const uint8_t *p2, float *x, float *attn_dump, DevState *st) {
    __shared__ uint32_t s_dig[128 * DIG_STRIDE];
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int ib = lane & 7, b0 = lane >> 3, b1 = 8 + (lane >> 3);
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    QXG_MARK(0, 0);
    DigIn<4096, false> din;
    digits_load(ctxv, nullptr, din);
    const float xr = lane < RPW ? x[r0 + lane] : 0.0f;
    uint4 q0[RPW], q1[RPW], q0b[RPW], q1b[RPW], h0a[RPW], h0b[RPW], h1a[RPW], h1b[RPW], m0[RPW], m1[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const uint64_t k0 = (uint64_t)(r0 + rr) * 16 + b0, k1 = (uint64_t)(r0 + rr) * 16 + b1;
        if constexpr (FMT == 23) {
            q0[rr] = ldw4(qs + k0 * 128 + 16 * ib);
            q1[rr] = ldw4(qs + k1 * 128 + 16 * ib);
            const uint2 a = ldw2(meta + k0 * 8), c = ldw2(meta + k1 * 8);
            m0[rr] = make_uint4(a.x, a.y, 0u, 0u);
            m1[rr] = make_uint4(c.x, c.y, 0u, 0u);
        } else {
            q0[rr] = ldw4(qs + k0 * 128 + 32 * (ib >> 1));
            q0b[rr] = ldw4(qs + k0 * 128 + 32 * (ib >> 1) + 16);
            q1[rr] = ldw4(qs + k1 * 128 + 32 * (ib >> 1));
            q1b[rr] = ldw4(qs + k1 * 128 + 32 * (ib >> 1) + 16);
            h0a[rr] = ldw4(p2 + k0 * 32);
            h0b[rr] = ldw4(p2 + k0 * 32 + 16);
            h1a[rr] = ldw4(p2 + k1 * 32);
            h1b[rr] = ldw4(p2 + k1 * 32 + 16);
            m0[rr] = ldw4(meta + k0 * 16);
            m1[rr] = ldw4(meta + k1 * 16);
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_ANCHOR(din.v[1][7]);
    QXG_MARK(0, 1);
    const bool ok = block_act<Q8>(din, s_dig, nullptr);
    QXG_MARK(0, 2);
    Dig g0, g1;
    load_dig(s_dig, lane, g0);
    load_dig(s_dig, lane + 64, g1);
    float part[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        if constexpr (FMT == 23)
            part[rr] = dot_iq4(q0[rr], make_uint2(m0[rr].x, m0[rr].y), ib, g0) +
                       dot_iq4(q1[rr], make_uint2(m1[rr].x, m1[rr].y), ib, g1);
        else
            part[rr] = dot_q5(q0[rr], q0b[rr], h0a[rr], h0b[rr], m0[rr], ib, g0) +
                       dot_q5(q1[rr], q1b[rr], h1a[rr], h1b[rr], m1[rr], ib, g1);
    }
    QXG_ANCHOR(part[0]); QXG_ANCHOR(part[RPW - 1]);
    QXG_MARK(0, 3);
    float out[RPW];
    rows_reduce<RPW>(part, out, lane);
    float mine = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) if (lane == rr) mine = out[rr];
    if (lane < RPW) {
        const int r = r0 + lane;
        const float o = (ok && isfinite(mine)) ? mine : 0.0f;
        if (attn_dump) attn_dump[r] = o;
        x[r] = xr + o;
    }
    if (Q8 && !ok && threadIdx.x == 0) st->q8_fault = QXG_Q8_NONFINITE_INPUT;
    QXG_MARK(0, 4);
}

// ffn RMSNorm + F32 router logits in double (reference src/qx_format.c:5254-5264);
// one workgroup per expert row, wave w taking values [512w, 512w + 512), 8 per lane
// (thread t holds values 8t..8t+7, the order of the other kernels' RMSNorm).  The
// softmax and top-8 run in the prologue of the gate/up kernel, where the ids are needed.
extern "C" __global__ __launch_bounds__(256) void qxk_router(const float *x, const float *norm_w, const float *router,
        uint32_t experts, double *logits) {
    __shared__ double s_ss[4], s_dot[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t e = blockIdx.x;   // grid = experts
    QXG_MARK(5, 0);
    const float4 *R = reinterpret_cast<const float4 *>(router + (uint64_t)e * 2048) + 2 * tid;
    const float4 *X = reinterpret_cast<const float4 *>(x) + 2 * tid;
    const float4 *W = reinterpret_cast<const float4 *>(norm_w) + 2 * tid;
    const float4 r0 = R[0], r1 = R[1], x0 = X[0], x1 = X[1], w0 = W[0], w1 = W[1];
    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const float r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_total_d(ss);
    if (lane == 0) s_ss[wave] = ss;
    __syncthreads();
    const double tot = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
    const double inv = 1.0 / sqrt(tot / 2048.0 + 1.0e-6);
    QXG_MARK(5, 1);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += (double)r[i] * (double)((float)((double)v[i] * inv) * w[i]);
    QXG_MARK(5, 2);
    acc = wave_total_d(acc);
    if (lane == 0) s_dot[wave] = acc;
    __syncthreads();
    if (tid == 0) logits[e] = (s_dot[0] + s_dot[1]) + (s_dot[2] + s_dot[3]);
    QXG_MARK(5, 3);
}
// gate/up (2048 -> 768; IQ2_XS, or IQ2_S in the real checkpoint) for the 8 routed experts
// (ids from st) + SwiGLU h[r][i] = (float)(silu((double)g) * (double)u)
// (src/qx_format.c:5298, 2511-2513).  Weight loads are issued first; the codebook tables
// go to LDS while they fly.  Units are processed in a rolled loop whose prefetch
// registers shift by one unit per iteration (static indices keep them in VGPRs).
// A unit's words: IQ2_XS {qs lo, qs hi, scale byte, d}; IQ2_S {grid bytes, sign bytes,
// qh | scale << 8, d}.
struct GuW {
    const uint8_t *qs, *p1, *p2;
    const uint16_t *d;
};

typedef uint32_t gu4 __attribute__((ext_vector_type(4)));   // register-promoted (a uint4 array is not)

template <int FMT>
DEV gu4 gu_load(const GuW &w, uint64_t blk, int ib) {
    gu4 r;
    if constexpr (FMT == 17) {
        const uint2 q = ldw2(w.qs + blk * 64 + 8 * ib);
        r.x = q.x; r.y = q.y; r.z = w.p1[blk * 8 + ib]; r.w = w.d[blk];
    } else {
        r.x = ldw1(w.qs + blk * 64 + 4 * ib);
        r.y = ldw1(w.qs + blk * 64 + 32 + 4 * ib);
        r.z = (uint32_t)w.p2[blk * 8 + ib] | ((uint32_t)w.p1[blk * 8 + ib] << 8);
        r.w = w.d[blk];
    }
    return r;
}

template <int FMT>
DEV float gu_dot(gu4 u, const Dig &g, const uint4 *G, const uint2 *SEL) {
    if constexpr (FMT == 17) return dot_iq2(make_uint2(u.x, u.y), u.z, u.w, g, G, SEL);
    else return dot_iq2s(u.x, u.y, u.z & 255u, u.z >> 8, u.w, g, G, SEL);
}

template <int UPW, int FMT, bool Q8>
__global__ __launch_bounds__(256) void qxk_gate_up(const float *x, const float *norm_w, GuW gw, GuW uw, Tables T,
        const double *logits, uint32_t experts, DevState *st, float *h, uint32_t *route_ids, double *route_w,
        const uint32_t *given_ids, float *gu_dump) {
    constexpr int NG = FMT == 17 ? 512 : 1024, NS = FMT == 17 ? 128 : 256;
    __shared__ uint4 s_g2[NG];
    __shared__ uint2 s_sel[NS];
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int b = lane >> 3, ib = lane & 7;
    const int u0 = (blockIdx.x * 4 + wave) * UPW;   // grid covers exactly 8*768 units
    const int E = (int)experts;
    QXG_MARK(1, 0);
    // the router logits head the longest chain (logits -> top-8 -> weights): loaded first;
    // every wave picks the experts itself (no barrier before its expert-row loads)
    const double l0 = lane < E ? logits[lane] : 0.0, l1 = lane + 64 < E ? logits[lane + 64] : 0.0;
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    const uint4 *G = FMT == 17 ? T.g2 : T.g2s;
    const uint2 *SL = FMT == 17 ? T.sel : T.sel8;
    gu4 tg[NG / 256];
#pragma unroll
    for (int i = 0; i < NG / 256; ++i) {
        const uint4 t = G[tid + 256 * i];
        tg[i].x = t.x; tg[i].y = t.y; tg[i].z = t.z; tg[i].w = t.w;
    }
    const uint2 t2 = SL[tid & (NS - 1)];
    uint32_t ids[QXG_TOPK];
    QXG_ANCHOR(l1);
    QXG_MARK(1, 5);
    if (given_ids) {   // the caller routed (st->moe_ids / moe_w already hold the picks)
#pragma unroll
        for (int q = 0; q < QXG_TOPK; ++q) ids[q] = given_ids[q];
    } else {
        wave_top8_ids(l0, l1, E, ids);
    }
    uint32_t e = 0u;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) {
        ids[q] = ids[q] < experts ? ids[q] : 0u;   // never address past the experts
        if (q == u0 / QXG_FFN) e = ids[q];           // UPW | 768: one expert per wave
    }
    QXG_MARK(1, 6);
    gu4 gq[UPW], uq[UPW];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
        const int i = (u0 + uu) % QXG_FFN;
        const uint64_t blk = ((uint64_t)e * QXG_FFN + i) * 8 + b;
        gq[uu] = gu_load<FMT>(gw, blk, ib);
        uq[uu] = gu_load<FMT>(uw, blk, ib);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    if (!given_ids && blockIdx.x == 0 && wave == 0) {   // the down kernel reads ids and renormalised weights from st
        double wts[QXG_TOPK];
        wave_top8_weights(l0, l1, ids, wts);
#pragma unroll
        for (int q = 0; q < QXG_TOPK; ++q)
            if (lane == q) {
                st->moe_ids[q] = ids[q];
                st->moe_w[q] = wts[q];
                route_ids[q] = ids[q];   // the layer's routing, kept for qxg_decode_routing
                route_w[q] = wts[q];
            }
    }
    QXG_MARK(1, 7);
#pragma unroll
    for (int i = 0; i < NG / 256; ++i) s_g2[tid + 256 * i] = make_uint4(tg[i].x, tg[i].y, tg[i].z, tg[i].w);
    if (tid < NS) s_sel[tid] = t2;
    QXG_ANCHOR(din.v[0][7]);
    QXG_MARK(1, 1);
    const bool ok = block_act<Q8>(din, s_dig, s_red);   // ends with a barrier
    QXG_MARK(1, 2);
    Dig g;
    load_dig(s_dig, lane, g);
    // dots unit by unit in a rolled loop (prefetch registers and results shift by one
    // slot per iteration, so every index is static), then one reduction for all units
    float pg[UPW], pu[UPW];
#pragma unroll 1
    for (int uu = 0; uu < UPW; ++uu) {
        const float a = gu_dot<FMT>(gq[0], g, s_g2, s_sel);
        const float c = gu_dot<FMT>(uq[0], g, s_g2, s_sel);
#pragma unroll
        for (int k = 0; k + 1 < UPW; ++k) {
            gq[k] = gq[k + 1]; uq[k] = uq[k + 1];
            pg[k] = pg[k + 1]; pu[k] = pu[k + 1];
        }
        pg[UPW - 1] = a;
        pu[UPW - 1] = c;
    }
    QXG_ANCHOR(pg[0]);
    QXG_MARK(1, 3);
    constexpr int R = 2 * UPW <= 2 ? 2 : (2 * UPW + 3) / 4 * 4;   // rows_reduce takes 2 or a multiple of 4
    float p[R], o[R];
#pragma unroll
    for (int k = 0; k < R; ++k) p[k] = 0.0f;
#pragma unroll
    for (int k = 0; k < UPW; ++k) { p[k] = pg[k]; p[UPW + k] = pu[k]; }
    rows_reduce<R>(p, o, lane);
    float gv = 0.0f, uv = 0.0f;
#pragma unroll
    for (int k = 0; k < UPW; ++k) if (lane == k) { gv = o[k]; uv = o[UPW + k]; }
    if (lane < UPW) {
        // q8_k_compat fails the step on a non-finite expert row (src/qx_format.c:4771)
        if (Q8 && (!ok || !isfinite(gv) || !isfinite(uv)))
            st->q8_fault = ok ? QXG_Q8_NONFINITE_EXPERT : QXG_Q8_NONFINITE_INPUT;
        gv = (ok && isfinite(gv)) ? gv : 0.0f;
        uv = (ok && isfinite(uv)) ? uv : 0.0f;
        if (gu_dump) {   // gate rows, then up rows, rank-major like h
            gu_dump[u0 + lane] = gv;
            gu_dump[QXG_TOPK * QXG_FFN + u0 + lane] = uv;
        }
        const double sg = (double)gv / (1.0 + exp(-(double)gv));
        h[u0 + lane] = (float)(sg * (double)uv);
    }
    QXG_MARK(1, 4);
}

// down (768 -> 2048; IQ3_XXS, or IQ4_XS / IQ3_S in the real checkpoint) for the 8 experts,
// rank-ordered weighted f32 sum and residual: x[i] = x[i] + sum_r (float)(w_r *
// (double)y_r[i]) (src/qx_format.c:5296-5309).  Wave per output row; lanes 8r..8r+7 hold
// rank r, lane 8r+k the sub-blocks k of blocks 0..2.  A sub-block's words: IQ3_XXS
// {qs lo, qs hi, aux, d}; IQ3_S {qs lo, qs hi, sign bytes, qh | scale << 8 | d << 16};
// IQ4_XS {qs (16 bytes)} + {meta (8 bytes)}.
struct DnW {
    const uint8_t *qs, *p1, *p2;
    const uint16_t *d;
};

template <int FMT>
DEV void dn_load(const DnW &w, uint64_t blk, int k, uint4 &a, uint2 &m) {
    if constexpr (FMT == 18) {
        const uint2 q = ldw2(w.qs + blk * 64 + 8 * k);
        a = make_uint4(q.x, q.y, ldw1(w.p1 + blk * 32 + 4 * k), w.d[blk]);
    } else if constexpr (FMT == 21) {
        const uint2 q = ldw2(w.qs + blk * 64 + 8 * k);
        const uint32_t sg = ldw1(w.p1 + blk * 32 + 4 * k);
        const uint32_t qh = w.p2[blk * 16 + k], sc = (w.p2[blk * 16 + 8 + (k >> 1)] >> (4 * (k & 1))) & 15u;
        a = make_uint4(q.x, q.y, sg, qh | (sc << 8) | ((uint32_t)w.d[blk] << 16));
    } else {
        a = ldw4(w.qs + blk * 128 + 16 * k);
        m = ldw2(w.p1 + blk * 8);
    }
}

template <int FMT>
DEV float dn_dot(uint4 a, uint2 m, int k, const Dig &g, const uint2 *G, const uint2 *SEL) {
    if constexpr (FMT == 18) return dot_iq3(make_uint2(a.x, a.y), a.z, a.w, g, G, SEL);
    else if constexpr (FMT == 21) return dot_iq3s(make_uint2(a.x, a.y), a.z, a.w & 255u, (a.w >> 8) & 255u, a.w >> 16, g, G, SEL);
    else return dot_iq4(a, m, k, g);
}

template <int RPW, int FMT, bool Q8>
__global__ __launch_bounds__(256) void qxk_down(const float *h, DnW w, Tables T, DevState *st, float *x,
                                                 float *moe_dump, float *down_dump, float *wdump) {
    constexpr int NG = FMT == 21 ? 512 : 256, NS = FMT == 21 ? 256 : 128;
    __shared__ uint2 s_g3[NG];
    __shared__ uint2 s_sel[NS];
    __shared__ uint32_t s_dig[192 * DIG_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int r = lane >> 3, k = lane & 7;
    const int r0 = (blockIdx.x * 4 + wave) * RPW;   // grid covers exactly 2048 rows
    QXG_MARK(2, 0);
    const uint32_t e = st->moe_ids[r];   // heads the id -> weights chain: loaded first
    double wr[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) wr[q] = st->moe_w[q];
    DigIn<QXG_TOPK * QXG_FFN, false> din;
    digits_load(h, nullptr, din);
    float xr[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) xr[rr] = x[r0 + rr];
    const uint2 *G = FMT == 21 ? T.g3s : T.g3;
    const uint2 *SL = FMT == 21 ? T.sel8 : T.sel;
    uint2 tg[NG / 256];
    if constexpr (FMT != 23) {
#pragma unroll
        for (int i = 0; i < NG / 256; ++i) tg[i] = G[tid + 256 * i];
    }
    const uint2 t1 = FMT != 23 ? SL[tid & (NS - 1)] : make_uint2(0u, 0u);
    uint4 qa[RPW][3];
    uint2 qm[RPW][3];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
        for (int j = 0; j < 3; ++j) dn_load<FMT>(w, ((uint64_t)e * 2048 + r0 + rr) * 3 + j, k, qa[rr][j], qm[rr][j]);
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    if constexpr (FMT != 23) {
#pragma unroll
        for (int i = 0; i < NG / 256; ++i) s_g3[tid + 256 * i] = tg[i];
        if (tid < NS) s_sel[tid] = t1;
    }
    QXG_ANCHOR(din.v[din.PER - 1][7]);
    QXG_MARK(2, 1);
    const bool ok = block_act<Q8>(din, s_dig, nullptr);   // ends with a barrier
    QXG_MARK(2, 2);
    Dig g[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) load_dig(s_dig, 24 * r + 8 * j + k, g[j]);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) part += dn_dot<FMT>(qa[rr][j], qm[rr][j], k, g[j], s_g3, s_sel);
        part += dppf<DPP_XOR1>(part);
        part += dppf<DPP_XOR2>(part);
        part += dppf<DPP_HALF_MIRROR>(part);   // lanes 8q..8q+7 now hold expert rank q's row
        if (Q8 && (!ok || !isfinite(part)) && k == 0)
            st->q8_fault = ok ? QXG_Q8_NONFINITE_EXPERT : QXG_Q8_NONFINITE_INPUT;
        const float y = (ok && isfinite(part)) ? part : 0.0f;
        if (down_dump && k == 0) {   // rank r's row and its weighted value, [rank][2048]
            down_dump[r * 2048 + r0 + rr] = y;
            wdump[r * 2048 + r0 + rr] = (float)(wr[r] * (double)y);
        }
        float moe = 0.0f;
#pragma unroll
        for (int q = 0; q < QXG_TOPK; ++q) moe += (float)(wr[q] * (double)rdlanef(y, 8 * q));
        if (lane == 0) {
            const int row = r0 + rr;
            if (moe_dump) moe_dump[row] = moe;
            x[row] = xr[rr] + moe;
        }
        if (rr == 0) QXG_MARK(2, 3);
    }
    QXG_MARK(2, 4);
}

// output RMSNorm + Q6_K head (2048 -> vocab) -> f32 logits (src/qx_format.c:3554-3738).
// Skipped on prompt steps unless forced.  A non-finite logit sets st->nonfinite.
// output RMSNorm + digits once per token into a global buffer (64 groups of
// DIG_STRIDE dwords, then the all-finite flag); the head waves load their group.
extern "C" __global__ __launch_bounds__(256) void qxk_norm_digits(const float *x, const float *norm_w, uint32_t *dig,
                                                                   float *norm_dump, DevState *st, uint32_t q8) {
    if (prompt_step(st)) return;
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    // q8_k_compat: Q8_K codes of the normed residual for the Q6_K head (src/qx_format.c:4026-4027)
    const bool ok = q8 ? block_q8(din, s_dig, s_red, norm_dump) : block_digits(din, s_dig, s_red, norm_dump);
    if (q8 && !ok && threadIdx.x == 0) st->q8_fault = QXG_Q8_NONFINITE_INPUT;
    for (int i = threadIdx.x; i < 64 * DIG_STRIDE; i += 256) dig[i] = s_dig[i];
    if (threadIdx.x == 0) dig[64 * DIG_STRIDE] = ok ? 1u : 0u;
}

// Q8_K blocks of n values (n a multiple of 256) in ggml's block_q8_K layout: f32 d, 256
// int8 codes, 16 int16 sums of 16 codes (src/qx_format.c:3891-3927).  Thread per 8
// values; a 256-value block is one half-wave.  *bad is set on a non-finite value.
extern "C" __global__ __launch_bounds__(256) void qxk_q8k(const float *x, uint32_t n, uint8_t *out, uint32_t *bad) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;   // chunk of 8 values
    const bool live = c < n / 8;                         // whole half-waves live or not (256 | n)
    float v[8];
    bool fin = true;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = live ? x[8 * c + i] : 0.0f;
        fin = fin && isfinite(v[i]);
    }
    uint32_t h0, h1;
    const float d = q8_chunk(v, h0, h1);
    int s8 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s8 += (int8_t)(((i < 4 ? h0 : h1) >> (8 * (i & 3))) & 255u);
    const int s16 = s8 + __shfl_xor(s8, 1);   // a 16-code sum spans the chunks 2j, 2j+1
    if (!live) return;
    uint8_t *blk = out + (uint64_t)(c / 32) * 292;
    const uint32_t k = c % 32;
    if (k == 0) *reinterpret_cast<float *>(blk) = d;
    reinterpret_cast<uint32_t *>(blk + 4)[2 * k] = h0;   // 292-byte blocks: dword alignment only
    reinterpret_cast<uint32_t *>(blk + 4)[2 * k + 1] = h1;
    if (!(k & 1)) *reinterpret_cast<int16_t *>(blk + 260 + k) = (int16_t)s16;
    if (!fin) *bad = 1u;
}

template <int RPW>
__global__ __launch_bounds__(256) void qxk_head(const uint32_t *dig, const uint8_t *ql,
        const uint8_t *qh, const int8_t *sc, const uint16_t *dd, uint32_t vocab, DevState *st, float *logits) {
    if (prompt_step(st)) return;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int b = lane >> 3, ib = lane & 7, hh = ib >> 2, k = ib & 3;
    const uint32_t r0 = (blockIdx.x * 4 + wave) * RPW;
    uint4 l0[RPW], l1[RPW], h0[RPW], h1[RPW];
    int s0[RPW], s1[RPW];
    uint32_t d16[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const uint32_t r = min(r0 + rr, vocab - 1);   // tail rows re-read the last row; not stored
        const uint64_t blk = (uint64_t)r * 8 + b;
        const uint8_t *lp = ql + blk * 128 + 64 * hh + 32 * (k & 1), *hp = qh + blk * 64 + 32 * hh;
        l0[rr] = ldw4(lp); l1[rr] = ldw4(lp + 16); h0[rr] = ldw4(hp); h1[rr] = ldw4(hp + 16);
        const int8_t *sp = sc + blk * 16 + 8 * hh + 2 * k;
        s0[rr] = sp[0]; s1[rr] = sp[1];
        d16[rr] = dd[blk];
    }
    Dig g;
    load_dig(dig, lane, g);
    const bool ok = dig[64 * DIG_STRIDE] != 0u;
    const Q6Bias bias = q6_bias(g);
    float part[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) part[rr] = dot_q6(l0[rr], l1[rr], h0[rr], h1[rr], s0[rr], s1[rr], d16[rr], ib, g, bias);
    float out[RPW];
    rows_reduce<RPW>(part, out, lane);
    float mine = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) if (lane == rr) mine = out[rr];
    if (lane < RPW && r0 + lane < vocab) {
        logits[r0 + lane] = mine;
        if (!ok || !isfinite(mine)) st->nonfinite = 1u;
    }
}

// top-N (N <= 32) over logits by (value desc, index asc): each block of qxk_topk
// reduces a slice to N candidates, qxk_topk_merge (one block, the next launch) merges
// them and writes tokens[step+1] = argmax on generate steps.  Round r picks the best element strictly below pick r-1 in that
// total order, so equal values are taken in index order.
namespace {
DEV bool better(float v, uint32_t i, float bv, uint32_t bi) { return v > bv || (v == bv && i < bi); }

DEV void block_best(float &v, uint32_t &i, float *sv, uint32_t *si) {
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const uint32_t oi = __shfl_xor(i, o);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = i; }
    __syncthreads();
    v = sv[0]; i = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
        if (better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
}

DEV void select_topn(const float *vals, const uint32_t *idx, uint32_t n, uint32_t topn, float *ov, uint32_t *oi,
                     float *sv, uint32_t *si) {
    float pv = INFINITY;
    uint32_t pi = 0;
    bool first = true;
    for (uint32_t r = 0; r < topn; ++r) {
        float bv = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
            const float v = vals[t];
            const uint32_t i = idx ? idx[t] : t;
            if (i == 0xffffffffu) continue;
            const bool below = first || better(pv, pi, v, i);
            if (below && better(v, i, bv, bi)) { bv = v; bi = i; }
        }
        block_best(bv, bi, sv, si);
        if (threadIdx.x == 0) { ov[r] = bv; oi[r] = bi; }
        pv = bv; pi = bi; first = false;
    }
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void qxk_topk(const float *logits, uint32_t vocab, uint32_t topn,
        float *cand_v, uint32_t *cand_i, float *top_v, uint32_t *top_i, uint32_t *tokens, DevState *st) {
    if (prompt_step(st)) return;
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const uint32_t chunk = (vocab + gridDim.x - 1) / gridDim.x;
    const uint32_t s0 = blockIdx.x * chunk, s1 = min(vocab, s0 + chunk);
    const uint32_t n = s1 > s0 ? s1 - s0 : 0;
    // local candidates (indices are global)
    {
        float pv = INFINITY;
        uint32_t pi = 0;
        for (uint32_t r = 0; r < topn; ++r) {
            float bv = -INFINITY;
            uint32_t bi = 0xffffffffu;
            for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
                const float v = logits[s0 + t];
                const uint32_t i = s0 + t;
                if ((r == 0 || better(pv, pi, v, i)) && better(v, i, bv, bi)) { bv = v; bi = i; }
            }
            block_best(bv, bi, sv, si);
            if (threadIdx.x == 0) { cand_v[blockIdx.x * topn + r] = bv; cand_i[blockIdx.x * topn + r] = bi; }
            pv = bv; pi = bi;
        }
    }
}
// the merge of qxk_topk's per-block candidates (one block; the kernel boundary makes
// them visible without fences), and tokens[step+1] = argmax on generate steps
extern "C" __global__ __launch_bounds__(256) void qxk_topk_merge(const float *cand_v, const uint32_t *cand_i,
        uint32_t blocks, uint32_t topn, float *top_v, uint32_t *top_i, uint32_t *tokens, DevState *st) {
    if (prompt_step(st)) return;
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    select_topn(cand_v, cand_i, blocks * topn, topn, top_v, top_i, sv, si);
    if (threadIdx.x == 0 && st->step + 1 >= st->n_prompt) tokens[st->step + 1] = top_i[0];
}

// Next step: step + 1, and the RoPE row of its position (64 threads)
extern "C" __global__ void qxk_advance(DevState *st, const double *rope_cos, const double *rope_sin) {
    const uint32_t step = st->step + 1, p = min(st->pos0 + step, (uint32_t)QXG_MAX_CTX - 1);
    const int i = threadIdx.x;
    st->rope_c[i] = rope_cos[p * 64 + i];
    st->rope_s[i] = rope_sin[p * 64 + i];
    if (i == 0) st->step = step;
}

// Bit-exact block dequant from the repacked planes (the reference's op order,
// src/qx_format.c:1914-2169): thread per value.
extern "C" __global__ __launch_bounds__(256) void qxk_dequant(uint32_t type, const uint8_t *p0, const uint8_t *p1,
        const uint8_t *p2, const uint16_t *dd, Tables T, uint64_t nblocks, float *out) {
    const uint64_t blk = blockIdx.x;
    if (blk >= nblocks) return;
    const int i = threadIdx.x;
    float y = 0.0f;
    if (type == 23) {
        const uint8_t *meta = p1 + blk * 8, *qs = p0 + blk * 128;
        const uint32_t sh = meta[2] | (meta[3] << 8);
        const int ib = i >> 5, j = i & 31;
        const int ls = ((meta[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = fp16_exact(meta[0] | (meta[1] << 8)) * (float)(ls - 32);
        const uint8_t q = qs[16 * ib + (j & 15)];
        y = dl * (float)KV[j < 16 ? (q & 15) : (q >> 4)];
    } else if (type == 17) {
        const int ib = i >> 5, l = (i >> 3) & 3, j = i & 7;
        const uint8_t s = p1[blk * 8 + ib];
        const float d = fp16_exact(dd[blk]);
        const float db = l < 2 ? (d * (0.5f + (float)(s & 15))) * 0.25f : (d * (0.5f + (float)(s >> 4))) * 0.25f;
        const uint16_t q = reinterpret_cast<const uint16_t *>(p0 + blk * 64)[4 * ib + l];
        const uint4 gg = T.g2[q & 511];
        const uint32_t gw = j < 4 ? gg.x : gg.y;
        const uint32_t gb = (gw >> (8 * (j & 3))) & 255;
        const uint32_t sgn = (uint32_t)(q >> 9) | ((uint32_t)(__popc(q >> 9) & 1) << 7);
        y = (db * (float)gb) * (((sgn >> j) & 1) ? -1.0f : 1.0f);
    } else if (type == 18) {
        const int ib = i >> 5, l = (i >> 3) & 3, j = i & 7;
        const uint32_t a = reinterpret_cast<const uint32_t *>(p1 + blk * 32)[ib];
        const float db = (fp16_exact(dd[blk]) * (0.5f + (float)(a >> 28))) * 0.5f;
        const uint32_t sidx = (a >> (7 * l)) & 127u;
        const uint32_t sgn = sidx | ((uint32_t)(__popc(sidx) & 1) << 7);
        const uint8_t gi = p0[blk * 64 + 8 * ib + 2 * l + (j >> 2)];
        const uint32_t gb = (T.g3[gi].x >> (8 * (j & 3))) & 255;
        y = (db * (float)gb) * (((sgn >> j) & 1) ? -1.0f : 1.0f);
    } else if (type == 14) {
        const int h = i >> 7, kk = (i >> 5) & 3, l = i & 31;
        const uint8_t qlb = p0[blk * 128 + 64 * h + l + 32 * (kk & 1)];
        const uint8_t qhb = p1[blk * 64 + 32 * h + l];
        const int q = (int)(((qlb >> (4 * (kk >> 1))) & 15) | (((qhb >> (2 * kk)) & 3) << 4)) - 32;
        const int8_t s = (int8_t)p2[blk * 16 + 8 * h + 2 * kk + (l >> 4)];
        y = (fp16_exact(dd[blk]) * (float)s) * (float)q;
    } else if (type == 12) {
        const uint8_t *b = p0 + blk * 144;
        const int j = i >> 6, hi = (i >> 5) & 1, l = i & 31;
        const int is = 2 * j + hi;
        const uint8_t *sc = b + 4;
        uint32_t s, m;
        if (is < 4) { s = sc[is] & 63u; m = sc[is + 4] & 63u; }
        else { s = (sc[is + 4] & 15u) | ((uint32_t)(sc[is - 4] >> 6) << 4); m = (sc[is + 4] >> 4) | ((uint32_t)(sc[is] >> 6) << 4); }
        const float d1 = fp16_exact(b[0] | (b[1] << 8)) * (float)s, m1 = fp16_exact(b[2] | (b[3] << 8)) * (float)m;
        const uint8_t q = b[16 + 32 * j + l];
        y = d1 * (float)(hi ? (q >> 4) : (q & 15)) - m1;
    } else if (type == 13) {
        const uint8_t *meta = p1 + blk * 16, *sc = meta + 4;
        const int j = i >> 6, hi = (i >> 5) & 1, l = i & 31;
        const int is = 2 * j + hi;
        uint32_t s, m;
        if (is < 4) { s = sc[is] & 63u; m = sc[is + 4] & 63u; }
        else { s = (sc[is + 4] & 15u) | ((uint32_t)(sc[is - 4] >> 6) << 4); m = (sc[is + 4] >> 4) | ((uint32_t)(sc[is] >> 6) << 4); }
        const float d1 = fp16_exact(meta[0] | (meta[1] << 8)) * (float)s, m1 = fp16_exact(meta[2] | (meta[3] << 8)) * (float)m;
        const uint8_t q = p0[blk * 128 + 32 * j + l];
        const uint32_t code = (hi ? (q >> 4) : (q & 15u)) | (((uint32_t)(p2[blk * 32 + l] >> is) & 1u) << 4);
        y = d1 * (float)code - m1;
    } else if (type == 22) {
        const int ib = i >> 5, l = (i >> 3) & 3, j = i & 7;
        const uint8_t s = p1[blk * 8 + ib];
        const float d = fp16_exact(dd[blk]);
        const float db = l < 2 ? (d * (0.5f + (float)(s & 15))) * 0.25f : (d * (0.5f + (float)(s >> 4))) * 0.25f;
        const uint32_t idx = (uint32_t)p0[blk * 64 + 4 * ib + l] | (((uint32_t)p2[blk * 8 + ib] << (8 - 2 * l)) & 0x300u);
        const uint4 gg = T.g2s[idx];
        const uint32_t gb = ((j < 4 ? gg.x : gg.y) >> (8 * (j & 3))) & 255u;
        const uint32_t sgn = p0[blk * 64 + 32 + 4 * ib + l];
        y = (db * (float)gb) * (((sgn >> j) & 1) ? -1.0f : 1.0f);
    } else if (type == 21) {
        const int ib = i >> 5, l = (i >> 3) & 3, j = i & 7;
        const uint8_t *ex = p2 + blk * 16;   // qh[8], scales[4]
        const uint32_t qh = ex[ib], sc = (ex[8 + ib / 2] >> (4 * (ib & 1))) & 15u;
        const float db = fp16_exact(dd[blk]) * (1.0f + 2.0f * (float)sc);
        const uint32_t gi = (j < 4) ? ((uint32_t)p0[blk * 64 + 8 * ib + 2 * l] | ((qh << (8 - 2 * l)) & 256u))
                                    : ((uint32_t)p0[blk * 64 + 8 * ib + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256u));
        const uint32_t gb = (T.g3s[gi].x >> (8 * (j & 3))) & 255u;
        const uint32_t sgn = p1[blk * 32 + 4 * ib + l];
        y = (db * (float)gb) * (((sgn >> j) & 1) ? -1.0f : 1.0f);
    }
    out[blk * 256 + i] = y;
}

// Split original blocks into the per-field arrays described in qxg_internal.h.
extern "C" __global__ __launch_bounds__(256) void qxk_repack(uint32_t type, const uint8_t *raw, uint64_t nblocks,
        uint8_t *p0, uint8_t *p1, uint8_t *p2, uint16_t *dd) {
    const uint64_t blk = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= nblocks) return;
    if (type == 23) {
        const uint8_t *b = raw + blk * 136;
        for (int i = 0; i < 8; ++i) p1[blk * 8 + i] = b[i];
        for (int i = 0; i < 128; ++i) p0[blk * 128 + i] = b[8 + i];
    } else if (type == 17) {
        const uint8_t *b = raw + blk * 74;
        dd[blk] = (uint16_t)(b[0] | (b[1] << 8));
        for (int i = 0; i < 64; ++i) p0[blk * 64 + i] = b[2 + i];
        for (int i = 0; i < 8; ++i) p1[blk * 8 + i] = b[66 + i];
    } else if (type == 18) {
        const uint8_t *b = raw + blk * 98;
        dd[blk] = (uint16_t)(b[0] | (b[1] << 8));
        for (int i = 0; i < 64; ++i) p0[blk * 64 + i] = b[2 + i];
        for (int i = 0; i < 32; ++i) p1[blk * 32 + i] = b[66 + i];
    } else if (type == 14) {
        const uint8_t *b = raw + blk * 210;
        for (int i = 0; i < 128; ++i) p0[blk * 128 + i] = b[i];
        for (int i = 0; i < 64; ++i) p1[blk * 64 + i] = b[128 + i];
        for (int i = 0; i < 16; ++i) p2[blk * 16 + i] = b[192 + i];
        dd[blk] = (uint16_t)(b[208] | (b[209] << 8));
    } else if (type == 13) {
        const uint8_t *b = raw + blk * 176;
        for (int i = 0; i < 16; ++i) p1[blk * 16 + i] = b[i];
        for (int i = 0; i < 32; ++i) p2[blk * 32 + i] = b[16 + i];
        for (int i = 0; i < 128; ++i) p0[blk * 128 + i] = b[48 + i];
    } else if (type == 22) {
        const uint8_t *b = raw + blk * 82;
        dd[blk] = (uint16_t)(b[0] | (b[1] << 8));
        for (int i = 0; i < 64; ++i) p0[blk * 64 + i] = b[2 + i];
        for (int i = 0; i < 8; ++i) p2[blk * 8 + i] = b[66 + i];
        for (int i = 0; i < 8; ++i) p1[blk * 8 + i] = b[74 + i];
    } else if (type == 21) {
        const uint8_t *b = raw + blk * 110;
        dd[blk] = (uint16_t)(b[0] | (b[1] << 8));
        for (int i = 0; i < 64; ++i) p0[blk * 64 + i] = b[2 + i];
        for (int i = 0; i < 8; ++i) p2[blk * 16 + i] = b[66 + i];
        for (int i = 0; i < 32; ++i) p1[blk * 32 + i] = b[74 + i];
        for (int i = 0; i < 4; ++i) p2[blk * 16 + 8 + i] = b[106 + i];
        for (int i = 0; i < 4; ++i) p2[blk * 16 + 12 + i] = 0;
    }
}

// MoE stage probe routing (reference src/qx_format.c:5647-5684), one thread, index order:
// f32 logits, f32 probabilities exp(logit - max) / sum (double max and sum), 8 picks by
// probability (strictly larger; the lowest index among equals), f32 weights and their
// double sum, f32 renormalised weights.  The picks and weights go to st for the expert
// kernels; out: logits[E], probs[E], topk[8], weights[8], weights_sum[1], weights_norm[8].
// *bad: 0, or the first of the reference's failures (1 non-finite logit, 2 invalid softmax,
// 3 invalid selected weights).
extern "C" __global__ void qxk_stage_route(const double *logits, uint32_t experts, float *out, DevState *st,
                                           uint32_t *bad) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const uint32_t E = experts;
    float *lg = out, *pr = out + E, *topk = pr + E, *wts = topk + 8, *wsum = wts + 8, *wn = wsum + 1;
    double mx = -1.0e300;
    uint32_t fail = 0u;
    for (uint32_t e = 0; e < E; ++e) {
        const double d = logits[e];
        if (!isfinite(d) && !fail) fail = 1u;   // 1: non-finite router logit
        lg[e] = (float)d;
        if (d > mx) mx = d;
    }
    double den = 0.0;
    for (uint32_t e = 0; e < E; ++e) { pr[e] = (float)exp((double)lg[e] - mx); den += (double)pr[e]; }
    if ((!isfinite(den) || den <= 0.0) && !fail) fail = 2u;   // 2: invalid softmax
    for (uint32_t e = 0; e < E; ++e) pr[e] = (float)((double)pr[e] / den);
    uint64_t picked[2] = {0ull, 0ull};
    double sum = 0.0;
    for (int r = 0; r < QXG_TOPK; ++r) {
        uint32_t best = 0u;
        float bp = -1.0f;
        for (uint32_t e = 0; e < E; ++e)
            if (!((picked[e >> 6] >> (e & 63)) & 1ull) && pr[e] > bp) { best = e; bp = pr[e]; }
        picked[best >> 6] |= 1ull << (best & 63);
        topk[r] = (float)best;
        wts[r] = bp;
        sum += (double)bp;
        st->moe_ids[r] = best;
    }
    if ((!isfinite(sum) || sum <= 0.0) && !fail) fail = 3u;   // 3: invalid selected weights
    wsum[0] = (float)sum;
    for (int r = 0; r < QXG_TOPK; ++r) {
        wn[r] = (float)((double)wts[r] / sum);
        st->moe_w[r] = (double)wn[r];   // the down kernel's weights: weighted = (float)(wn * down)
    }
    *bad = fail;
}

// The attention stage probe's context (reference src/qx_format.c:5532-5539): a single token
// attends to itself with weight 1, so q head h's context is kv head h/8's V row (with
// fp16 KV, after an fp16 round trip: round to nearest even, the reference's conversion).
extern "C" __global__ __launch_bounds__(256) void qxk_stage_ctx(const float *qkv, uint32_t f16, float *ctxv) {
    for (uint32_t i = threadIdx.x; i < 4096; i += 256) {
        const float v = qkv[4608 + ((i >> 10) << 7) + (i & 127)];
        ctxv[i] = f16 ? (float)(_Float16)v : v;
    }
}

// ----------------------------------------------------------------- launch wrappers
extern "C" {
// Each wrapper picks the kernel instantiation of the tensor's format (validated at bind)
// and of the activation mode (q8: q8_k_compat).
void qxl_qkv(hipStream_t s, const float *x, const float *nw, const QTensor *q, const QTensor *k, const QTensor *v, float *qkv,
             DevState *st, bool q8, Timer t) {
    QkvW w;
    const QTensor *m[3] = {q, k, v};
    for (int i = 0; i < 3; ++i) { w.qs[i] = m[i]->p0; w.p1[i] = m[i]->p1; w.p2[i] = m[i]->p2; w.type[i] = m[i]->type; }
    if (q8) qx_launch(qxk_qkv<true>, dim3(512), dim3(256), 0, s, t, x, nw, w, qkv, st);
    else qx_launch(qxk_qkv<false>, dim3(512), dim3(256), 0, s, t, x, nw, w, qkv, st);
}
void qxl_oproj(hipStream_t s, const float *ctxv, const QTensor *o, float *x, float *dump, DevState *st, bool q8, Timer t) {
    constexpr int RPW = QXG_OPROJ_RPW;
    const dim3 grid(2048 / (4 * RPW));
    auto go = [&](auto kernel) { qx_launch(kernel, grid, dim3(256), 0, s, t, ctxv, o->p0, o->p1, o->p2, x, dump, st); };
    if (o->type == 13) q8 ? go(qxk_oproj<RPW, 13, true>) : go(qxk_oproj<RPW, 13, false>);
    else q8 ? go(qxk_oproj<RPW, 23, true>) : go(qxk_oproj<RPW, 23, false>);
}
void qxl_gate_up(hipStream_t s, const float *x, const float *nw, const QTensor *g, const QTensor *u, Tables T,
                 const double *logits, uint32_t experts, DevState *st, float *h, uint32_t *route_ids, double *route_w,
                 bool q8, Timer t, const uint32_t *given_ids, float *gu_dump) {
    constexpr int UPW = QXG_GU_UPW;
    const GuW gw{g->p0, g->p1, g->p2, g->d}, uw{u->p0, u->p1, u->p2, u->d};
    const dim3 grid(QXG_TOPK * QXG_FFN / (4 * UPW));
    auto go = [&](auto kernel) {
        qx_launch(kernel, grid, dim3(256), 0, s, t, x, nw, gw, uw, T, logits, experts, st, h, route_ids, route_w,
                  given_ids, gu_dump);
    };
    if (g->type == 22) q8 ? go(qxk_gate_up<UPW, 22, true>) : go(qxk_gate_up<UPW, 22, false>);
    else q8 ? go(qxk_gate_up<UPW, 17, true>) : go(qxk_gate_up<UPW, 17, false>);
}
void qxl_down(hipStream_t s, const float *h, const QTensor *d, Tables T, DevState *st, float *x, float *dump, bool q8, Timer t,
              float *down_dump, float *wdump) {
    constexpr int RPW = QXG_DOWN_RPW;
    const DnW w{d->p0, d->p1, d->p2, d->d};
    const dim3 grid(2048 / (4 * RPW));
    auto go = [&](auto kernel) { qx_launch(kernel, grid, dim3(256), 0, s, t, h, w, T, st, x, dump, down_dump, wdump); };
    if (d->type == 23) q8 ? go(qxk_down<RPW, 23, true>) : go(qxk_down<RPW, 23, false>);
    else if (d->type == 21) q8 ? go(qxk_down<RPW, 21, true>) : go(qxk_down<RPW, 21, false>);
    else q8 ? go(qxk_down<RPW, 18, true>) : go(qxk_down<RPW, 18, false>);
}
void qxl_head(hipStream_t s, const float *x, const float *nw, const QTensor *w, uint32_t vocab, DevState *st,
              float *logits, float *norm_dump, uint32_t *dig, bool q8, Timer t) {
    constexpr int RPW = 2;   // rows per wave (measured: 2 rows 0.8 % faster per token than 4, 8 no better)
    hipLaunchKernelGGL(qxk_norm_digits, dim3(1), dim3(256), 0, s, x, nw, dig, norm_dump, st, (uint32_t)q8);
    const uint32_t grid = (vocab + 4 * RPW - 1) / (4 * RPW);
    qx_launch(qxk_head<RPW>, dim3(grid), dim3(256), 0, s, t, dig, w->p0, w->p1, (const int8_t *)w->p2, w->d,
                       vocab, st, logits);
}
}
