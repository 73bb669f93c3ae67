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
#include "qxg_internal.h"

#define DEV __device__ __forceinline__

namespace {

// ---------------------------------------------------------------- helpers
// reference qx_fp16_to_f32 (src/qx_format.c:1854-1876): exact, exponent 31 -> +-65504
DEV float fp16_exact(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            int sh = __builtin_clz(m) - 21;          // shifts until bit 10 is set
            bits = sign | ((uint32_t)(113 - sh) << 23) | (((m << sh) & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x477fe000u;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

DEV double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// 32 activations of one group as three int8 digit planes and a power-of-two scale
struct Dig {
    uint32_t h[8], m[8], l[8];
    float s;
};

// returns false if any value is non-finite
DEV bool make_digits(const float *v, Dig &g) {
    float mx = 0.0f;
    bool fin = true;
#pragma unroll
    for (int i = 0; i < 32; ++i) { fin = fin && isfinite(v[i]); mx = fmaxf(mx, fabsf(v[i])); }
    int e = 0;
    if (fin && mx > 0.0f) (void)frexpf(mx, &e);   // 2^(e-1) <= mx < 2^e
    else if (!fin) mx = 0.0f;
    g.s = mx > 0.0f ? ldexpf(1.0f, e - 22) : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t ph = 0, pm = 0, pl = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int X = mx > 0.0f ? (int)rintf(ldexpf(v[4 * k + j], 22 - e)) : 0;  // |X| <= 2^22
            int L = ((X + 128) & 255) - 128;
            int X1 = (X - L) >> 8;
            int M = ((X1 + 128) & 255) - 128;
            int H = (X1 - M) >> 8;
            ph |= (uint32_t)(H & 255) << (8 * j);
            pm |= (uint32_t)(M & 255) << (8 * j);
            pl |= (uint32_t)(L & 255) << (8 * j);
        }
        g.h[k] = ph; g.m[k] = pm; g.l[k] = pl;
    }
    return fin;
}

DEV float combine(int aH, int aM, int aL) {
    return fmaf((float)aH, 65536.0f, fmaf((float)aM, 256.0f, (float)aL));
}

// IQ4_XS codebook (reference qx_kvalues_iq4nl, src/qx_format.c:2032) as 4 byte-lanes
constexpr int8_t KV[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
constexpr uint32_t kvw(int i) {
    return (uint32_t)(uint8_t)KV[i] | ((uint32_t)(uint8_t)KV[i + 1] << 8) | ((uint32_t)(uint8_t)KV[i + 2] << 16) |
           ((uint32_t)(uint8_t)KV[i + 3] << 24);
}

// 4 nibbles (one per byte, values 0..15) -> 4 signed codebook bytes
DEV uint32_t kv_lookup(uint32_t n) {
    const uint32_t n7 = n & 0x07070707u;
    const uint32_t lo = perm(kvw(4), kvw(0), n7);
    const uint32_t hi = perm(kvw(12), kvw(8), n7);
    return perm(hi, lo, ((n >> 1) & 0x04040404u) | 0x03020100u);
}

// ---------------------------------------------------------------- per-format sub-block dots
// IQ4_XS sub-block ib (32 values): codes kvalue[nibble], scale d*(ls-32)
DEV float dot_iq4(uint4 qs, uint2 meta, int ib, const Dig &g) {
    const uint32_t sh = meta.x >> 16, sl = meta.y;
    const int ls = ((sl >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
    const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    int aH = 0, aM = 0, aL = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t wlo = kv_lookup(q[k] & 0x0f0f0f0fu);
        const uint32_t whi = kv_lookup((q[k] >> 4) & 0x0f0f0f0fu);
        aH = sdot4(wlo, g.h[k], aH); aH = sdot4(whi, g.h[4 + k], aH);
        aM = sdot4(wlo, g.m[k], aM); aM = sdot4(whi, g.m[4 + k], aM);
        aL = sdot4(wlo, g.l[k], aL); aL = sdot4(whi, g.l[4 + k], aL);
    }
    const float dl = fp16_exact(meta.x & 0xffffu) * (float)(ls - 32);
    return (dl * g.s) * combine(aH, aM, aL);
}

// IQ2_XS sub-block (32 values = 4 grid entries of 8): halves scaled d*(2s+1)/8
DEV float dot_iq2(uint2 qs, uint32_t sc, uint32_t d16, const Dig &g, const uint4 *G2, const uint2 *SEL) {
    const uint32_t qv[4] = {qs.x & 0xffffu, qs.x >> 16, qs.y & 0xffffu, qs.y >> 16};
    int h0 = 0, m0 = 0, l0 = 0, h1 = 0, m1 = 0, l1 = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint4 gg = G2[qv[l] & 511u];
        const uint2 sl = SEL[qv[l] >> 9];
        const uint32_t w0 = perm(gg.z, gg.x, sl.x), w1 = perm(gg.w, gg.y, sl.y);
        if (l < 2) {
            h0 = sdot4(w0, g.h[2 * l], h0); h0 = sdot4(w1, g.h[2 * l + 1], h0);
            m0 = sdot4(w0, g.m[2 * l], m0); m0 = sdot4(w1, g.m[2 * l + 1], m0);
            l0 = sdot4(w0, g.l[2 * l], l0); l0 = sdot4(w1, g.l[2 * l + 1], l0);
        } else {
            h1 = sdot4(w0, g.h[2 * l], h1); h1 = sdot4(w1, g.h[2 * l + 1], h1);
            m1 = sdot4(w0, g.m[2 * l], m1); m1 = sdot4(w1, g.m[2 * l + 1], m1);
            l1 = sdot4(w0, g.l[2 * l], l1); l1 = sdot4(w1, g.l[2 * l + 1], l1);
        }
    }
    const int k0 = 2 * (int)(sc & 15u) + 1, k1 = 2 * (int)(sc >> 4) + 1;
    const float v = combine(k0 * h0 + k1 * h1, k0 * m0 + k1 * m1, k0 * l0 + k1 * l1);
    return ((fp16_exact(d16) * 0.125f) * g.s) * v;
}

// IQ3_XXS sub-block: 8 grid indices (4 values each), scale d*(2a+1)/4
DEV float dot_iq3(uint2 qs, uint32_t aux, uint32_t d16, const Dig &g, const uint2 *G3, const uint2 *SEL) {
    int aH = 0, aM = 0, aL = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t word = l < 2 ? qs.x : qs.y;
        const uint32_t b1 = (word >> (16 * (l & 1))) & 255u, b2 = (word >> (16 * (l & 1) + 8)) & 255u;
        const uint2 g1 = G3[b1], g2 = G3[b2];
        const uint2 sl = SEL[(aux >> (7 * l)) & 127u];
        const uint32_t w0 = perm(g1.y, g1.x, sl.x), w1 = perm(g2.y, g2.x, sl.y);
        aH = sdot4(w0, g.h[2 * l], aH); aH = sdot4(w1, g.h[2 * l + 1], aH);
        aM = sdot4(w0, g.m[2 * l], aM); aM = sdot4(w1, g.m[2 * l + 1], aM);
        aL = sdot4(w0, g.l[2 * l], aL); aL = sdot4(w1, g.l[2 * l + 1], aL);
    }
    const int k = 2 * (int)(aux >> 28) + 1;
    return ((fp16_exact(d16) * 0.25f) * g.s) * combine(k * aH, k * aM, k * aL);
}

// Q6_K sub-block ib: values 128h+32k+l (h=ib/4, k=ib%4), two 16-value scale segments.
// Codes are taken unsigned (0..63); the -32 offset enters through the digit
// sums bias[seg] = -32 * sum(digits of the segment), precomputed per lane.
struct Q6Bias { int h[2], m[2], l[2]; };

DEV Q6Bias q6_bias(const Dig &g) {
    Q6Bias b;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int sh = 0, sm = 0, sl = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sh = sdot4(0x01010101u, g.h[4 * s + k], sh);
            sm = sdot4(0x01010101u, g.m[4 * s + k], sm);
            sl = sdot4(0x01010101u, g.l[4 * s + k], sl);
        }
        b.h[s] = -32 * sh; b.m[s] = -32 * sm; b.l[s] = -32 * sl;
    }
    return b;
}

DEV float dot_q6(uint4 ql0, uint4 ql1, uint4 qh0, uint4 qh1, int sc0, int sc1, uint32_t d16, int ib,
                 const Dig &g, const Q6Bias &bias) {
    const int k = ib & 3;
    const uint32_t shl = 4 * (k >> 1), shh = 2 * k;
    const uint32_t ql[8] = {ql0.x, ql0.y, ql0.z, ql0.w, ql1.x, ql1.y, ql1.z, ql1.w};
    const uint32_t qh[8] = {qh0.x, qh0.y, qh0.z, qh0.w, qh1.x, qh1.y, qh1.z, qh1.w};
    int aH[2] = {bias.h[0], bias.h[1]}, aM[2] = {bias.m[0], bias.m[1]}, aL[2] = {bias.l[0], bias.l[1]};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t u = ((ql[j] >> shl) & 0x0f0f0f0fu) | (((qh[j] >> shh) & 0x03030303u) << 4);
        const int s = j >> 2;
        aH[s] = sdot4(u, g.h[j], aH[s]);
        aM[s] = sdot4(u, g.m[j], aM[s]);
        aL[s] = sdot4(u, g.l[j], aL[s]);
    }
    const float v = combine(sc0 * aH[0] + sc1 * aH[1], sc0 * aM[0] + sc1 * aM[1], sc0 * aL[0] + sc1 * aL[1]);
    return (fp16_exact(d16) * g.s) * v;
}

// ---------------------------------------------------------------- prologues
// reference qx_apply_f32_rmsnorm (src/qx_format.c:3358-3371): double sum of
// squares, rms = sqrt(ss/n + 1e-6), y = (float)(x/rms) * w.  Lane handles the
// 32 values [32*lane, 32*lane+32) of a 2048-vector; the wave reduces.
DEV bool norm_digits_2048(const float *x, const float *w, int lane, Dig &g) {
    float v[32];
    const float4 *xp = reinterpret_cast<const float4 *>(x + 32 * lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = xp[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 32; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_sum_d(ss);
    const double rms = sqrt(ss / 2048.0 + 1.0e-6);
    const float4 *wp = reinterpret_cast<const float4 *>(w + 32 * lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = wp[i];
        v[4 * i] = (float)((double)v[4 * i] / rms) * t.x;
        v[4 * i + 1] = (float)((double)v[4 * i + 1] / rms) * t.y;
        v[4 * i + 2] = (float)((double)v[4 * i + 2] / rms) * t.z;
        v[4 * i + 3] = (float)((double)v[4 * i + 3] / rms) * t.w;
    }
    return make_digits(v, g);
}

DEV bool plain_digits(const float *x, Dig &g) {
    float v[32];
    const float4 *xp = reinterpret_cast<const float4 *>(x);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = xp[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    return make_digits(v, g);
}

DEV bool wave_all(bool b) { return __all(b) != 0; }

DEV void load_g2(uint4 *s_g2, uint2 *s_sel, const Tables &T) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) s_g2[i] = T.g2[i];
    for (int i = threadIdx.x; i < 128; i += blockDim.x) s_sel[i] = T.sel[i];
}

DEV uint32_t cur_pos(const DevState *st) { return st->pos0 + st->step; }

}  // namespace

// ================================================================= kernels

// Q4_K embedding row of tokens[step] -> x (reference src/qx_format.c:2079-2110,
// 3759-3793).  256 threads, thread (b, l) produces 8 values of block b.
extern "C" __global__ __launch_bounds__(256) void qxk_embed(const uint8_t *emb, uint64_t row_bytes,
                                                            const uint32_t *tokens, const DevState *st, float *x) {
    const uint32_t tok = tokens[st->step];
    const uint8_t *row = emb + (uint64_t)tok * row_bytes;
    const int b = threadIdx.x >> 5, l = threadIdx.x & 31;
    const uint8_t *blk = row + 144 * b;
    const float d = fp16_exact(blk[0] | (blk[1] << 8)), dmin = fp16_exact(blk[2] | (blk[3] << 8));
    const uint8_t *sc = blk + 4, *q = blk + 16;
    for (int j = 0; j < 4; ++j) {
        uint32_t s0, m0, s1, m1;
        const int i0 = 2 * j, i1 = 2 * j + 1;
        if (i0 < 4) { s0 = sc[i0] & 63u; m0 = sc[i0 + 4] & 63u; }
        else { s0 = (sc[i0 + 4] & 15u) | ((uint32_t)(sc[i0 - 4] >> 6) << 4); m0 = (sc[i0 + 4] >> 4) | ((uint32_t)(sc[i0] >> 6) << 4); }
        if (i1 < 4) { s1 = sc[i1] & 63u; m1 = sc[i1 + 4] & 63u; }
        else { s1 = (sc[i1 + 4] & 15u) | ((uint32_t)(sc[i1 - 4] >> 6) << 4); m1 = (sc[i1 + 4] >> 4) | ((uint32_t)(sc[i1] >> 6) << 4); }
        const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
        const uint8_t qq = q[32 * j + l];
        x[256 * b + 64 * j + l] = d1 * (float)(qq & 15) - mm1;
        x[256 * b + 64 * j + 32 + l] = d2 * (float)(qq >> 4) - mm2;
    }
}

// attn RMSNorm + Q/K/V IQ4_XS projections (2048 -> 4096 | 512 | 512) into qkv[5120].
// Wave per RPW consecutive rows; lane = 8*block + sub-block.
template <int RPW>
__global__ __launch_bounds__(256) void qxk_qkv(const float *x, const float *norm_w,
        const uint8_t *q_qs, const uint8_t *q_meta, const uint8_t *k_qs, const uint8_t *k_meta,
        const uint8_t *v_qs, const uint8_t *v_meta, float *qkv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 3, ib = lane & 7;
    Dig g;
    const bool ok = wave_all(norm_digits_2048(x, norm_w, lane, g));
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    for (int rr = 0; rr < RPW; ++rr) {
        const int r = r0 + rr;
        if (r >= 5120) break;
        const uint8_t *qs, *meta;
        int lr;
        if (r < 4096) { qs = q_qs; meta = q_meta; lr = r; }
        else if (r < 4608) { qs = k_qs; meta = k_meta; lr = r - 4096; }
        else { qs = v_qs; meta = v_meta; lr = r - 4608; }
        const uint64_t blk = (uint64_t)lr * 8 + b;
        const uint4 qv = reinterpret_cast<const uint4 *>(qs + blk * 128)[ib];
        const uint2 mv = *reinterpret_cast<const uint2 *>(meta + blk * 8);
        const float s = wave_sum(dot_iq4(qv, mv, ib, g));
        if (lane == 0) qkv[r] = (ok && isfinite(s)) ? s : 0.0f;
    }
}

// per-head q/k RMSNorm (src/qx_format.c:3740-3757) + split-half RoPE (4625-4641,
// cos/sin from the host-computed table) + INT8 K/V quantize (4449-4463) and store
// at [layer][pos].  Blocks 0..31: q heads; block 32: k heads then K/V quantize.
namespace {
DEV double block_sum_d128(double v, double *red) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1];
}

DEV void head_norm_rope(float *p, const float *w, uint32_t pos, const Tables &T, double *red, float *sv) {
    const int d = threadIdx.x;
    const float v = p[d];
    const double ss = block_sum_d128((double)v * (double)v, red);
    const double inv = 1.0 / sqrt(ss / 128.0 + 1.0e-6);
    sv[d] = (float)((double)v * inv * (double)w[d]);
    __syncthreads();
    if (d < 64) {
        const double c = T.rope_cos[pos * 64 + d], s = T.rope_sin[pos * 64 + d];
        const float x0 = sv[d], x1 = sv[d + 64];
        p[d] = (float)((double)x0 * c - (double)x1 * s);
        p[d + 64] = (float)((double)x0 * s + (double)x1 * c);
    }
    __syncthreads();
}

DEV void quantize512(const float *src, int8_t *dst, float *scale_out, float *red) {
    float mx = 0.0f;
    for (int i = threadIdx.x; i < 512; i += 128) {
        const float a = isfinite(src[i]) ? fabsf(src[i]) : 0.0f;
        mx = fmaxf(mx, a);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(red[0], red[1]);
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
    for (int i = threadIdx.x; i < 512; i += 128) {
        int q = isfinite(src[i]) ? (int)rintf(src[i] / scale) : 0;
        q = q < -127 ? -127 : q > 127 ? 127 : q;
        dst[i] = (int8_t)q;
    }
    if (threadIdx.x == 0) *scale_out = scale;
    __syncthreads();
}
}  // namespace

extern "C" __global__ __launch_bounds__(128) void qxk_qk_rope_kv(float *qkv, const float *q_norm, const float *k_norm,
        Tables T, int8_t *kc, int8_t *vc, float *ks, float *vs, uint32_t layer, uint32_t ctx, const DevState *st,
        float *vcur_dump) {
    __shared__ double red[2];
    __shared__ float redf[2];
    __shared__ float sv[128];
    const uint32_t pos = cur_pos(st);
    if (blockIdx.x < 32) {
        head_norm_rope(qkv + 128 * blockIdx.x, q_norm, pos, T, red, sv);
        return;
    }
    for (int h = 0; h < 4; ++h) head_norm_rope(qkv + 4096 + 128 * h, k_norm, pos, T, red, sv);
    const uint64_t slot = (uint64_t)layer * ctx + pos;
    quantize512(qkv + 4096, kc + slot * 512, ks + slot, redf);
    quantize512(qkv + 4608, vc + slot * 512, vs + slot, redf);
    if (vcur_dump)
        for (int i = threadIdx.x; i < 512; i += 128) vcur_dump[i] = qkv[4608 + i];
}

// GQA decode attention (reference src/qx_format.c:5127-5172): block per q head,
// double scores over positions 0..pos, double softmax, context accumulated in
// f32 per position (position order kept within each of NCH position chunks).
extern "C" __global__ __launch_bounds__(512) void qxk_attn(const float *qkv, const int8_t *kc, const int8_t *vc,
        const float *ks, const float *vs, uint32_t layer, uint32_t ctx, double inv_sqrt_divisor, const DevState *st,
        float *ctx_out) {
    extern __shared__ double s_sc[];
    __shared__ double s_q[128];
    __shared__ double red[8];
    __shared__ float s_part[4][128];
    const int tid = threadIdx.x;
    const int qh = blockIdx.x, kvh = qh >> 3;
    const uint32_t n = cur_pos(st) + 1;
    const uint64_t base = (uint64_t)layer * ctx;
    if (tid < 128) s_q[tid] = (double)qkv[qh * 128 + tid];
    __syncthreads();
    double mx = -1.0e300;
    for (uint32_t t = tid; t < n; t += 512) {
        const int8_t *kp = kc + (base + t) * 512 + kvh * 128;
        const float ksc = ks[base + t];
        double s = 0.0;
        for (int c = 0; c < 8; ++c) {
            const int4 kk = reinterpret_cast<const int4 *>(kp)[c];
            const int w[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int8_t kb = (int8_t)((w[j >> 2] >> (8 * (j & 3))) & 255);
                s += s_q[16 * c + j] * (double)((float)kb * ksc);
            }
        }
        s = s / inv_sqrt_divisor;
        if (!isfinite(s)) s = 0.0;
        s_sc[t] = s;
        mx = fmax(mx, s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < 8; ++i) mx = fmax(mx, red[i]);
    __syncthreads();
    double den = 0.0;
    for (uint32_t t = tid; t < n; t += 512) {
        const double e = exp(s_sc[t] - mx);
        s_sc[t] = e;
        den += e;
    }
    den = wave_sum_d(den);
    if ((tid & 63) == 0) red[tid >> 6] = den;
    __syncthreads();
    den = 0.0;
    for (int i = 0; i < 8; ++i) den += red[i];
    if (!isfinite(den) || den <= 0.0) den = 1.0;
    const int nch = n <= 128 ? 1 : 4;
    const int d = tid & 127, c = tid >> 7;
    if (c < nch) {
        const uint32_t t0 = (uint32_t)(((uint64_t)n * c) / nch), t1 = (uint32_t)(((uint64_t)n * (c + 1)) / nch);
        float acc = 0.0f;
        for (uint32_t t = t0; t < t1; ++t) {
            const double w = s_sc[t] / den;
            const float vv = (float)vc[(base + t) * 512 + kvh * 128 + d] * vs[base + t];
            acc += (float)(w * (double)vv);
        }
        s_part[c][d] = acc;
    }
    __syncthreads();
    if (tid < 128) {
        float out = s_part[0][tid];
        for (int i = 1; i < nch; ++i) out += s_part[i][tid];
        ctx_out[qh * 128 + tid] = out;
    }
}

// O projection IQ4_XS 4096 -> 2048 on ctx, then x[r] += o[r] (src/qx_format.c:6420-6423).
// Lane handles sub-blocks lane and lane+64 (blocks lane/8 and 8+lane/8).
template <int RPW>
__global__ __launch_bounds__(256) void qxk_oproj(const float *ctxv, const uint8_t *qs, const uint8_t *meta,
                                                  float *x, float *attn_dump) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ib = lane & 7, b0 = lane >> 3, b1 = 8 + (lane >> 3);
    Dig g0, g1;
    const bool f0 = plain_digits(ctxv + 32 * lane, g0);
    const bool f1 = plain_digits(ctxv + 32 * (lane + 64), g1);
    const bool ok = wave_all(f0 && f1);
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    for (int rr = 0; rr < RPW; ++rr) {
        const int r = r0 + rr;
        if (r >= 2048) break;
        const uint64_t k0 = (uint64_t)r * 16 + b0, k1 = (uint64_t)r * 16 + b1;
        const uint4 q0 = reinterpret_cast<const uint4 *>(qs + k0 * 128)[ib];
        const uint4 q1 = reinterpret_cast<const uint4 *>(qs + k1 * 128)[ib];
        const uint2 m0 = *reinterpret_cast<const uint2 *>(meta + k0 * 8);
        const uint2 m1 = *reinterpret_cast<const uint2 *>(meta + k1 * 8);
        const float s = wave_sum(dot_iq4(q0, m0, ib, g0) + dot_iq4(q1, m1, ib, g1));
        if (lane == 0) {
            const float o = (ok && isfinite(s)) ? s : 0.0f;
            if (attn_dump) attn_dump[r] = o;
            x[r] = x[r] + o;
        }
    }
}

// ffn RMSNorm + F32 router (double dot) over E experts; the last block to finish
// does the double softmax, top-8 (strict >, lowest index on ties) and the
// renormalisation (reference src/qx_format.c:5254-5285).  Wave per expert row.
extern "C" __global__ __launch_bounds__(256) void qxk_router(const float *x, const float *norm_w, const float *router,
        uint32_t experts, double *logits, DevState *st) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float v[32];
    {
        const float4 *xp = reinterpret_cast<const float4 *>(x + 32 * lane);
        for (int i = 0; i < 8; ++i) { const float4 t = xp[i]; v[4*i] = t.x; v[4*i+1] = t.y; v[4*i+2] = t.z; v[4*i+3] = t.w; }
        double ss = 0.0;
        for (int i = 0; i < 32; ++i) ss += (double)v[i] * (double)v[i];
        ss = wave_sum_d(ss);
        const double rms = sqrt(ss / 2048.0 + 1.0e-6);
        const float4 *wp = reinterpret_cast<const float4 *>(norm_w + 32 * lane);
        for (int i = 0; i < 8; ++i) {
            const float4 t = wp[i];
            v[4*i] = (float)((double)v[4*i] / rms) * t.x; v[4*i+1] = (float)((double)v[4*i+1] / rms) * t.y;
            v[4*i+2] = (float)((double)v[4*i+2] / rms) * t.z; v[4*i+3] = (float)((double)v[4*i+3] / rms) * t.w;
        }
    }
    const uint32_t e = blockIdx.x * 4 + wave;
    if (e < experts) {
        const float4 *rp = reinterpret_cast<const float4 *>(router + (uint64_t)e * 2048 + 32 * lane);
        double acc = 0.0;
        for (int i = 0; i < 8; ++i) {
            const float4 t = rp[i];
            acc += (double)t.x * (double)v[4*i]; acc += (double)t.y * (double)v[4*i+1];
            acc += (double)t.z * (double)v[4*i+2]; acc += (double)t.w * (double)v[4*i+3];
        }
        acc = wave_sum_d(acc);
        if (lane == 0) logits[e] = acc;
    }
    __shared__ uint32_t ticket;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) ticket = atomicAdd(&st->ctr_router, 1u);
    __syncthreads();
    if (ticket != gridDim.x - 1 || wave != 0) return;
    __threadfence();
    // one wave: lane holds experts lane and lane+64
    const volatile double *lg = logits;
    double p0 = lane < (int)experts ? lg[lane] : -1.0e300;
    double p1 = lane + 64 < (int)experts ? lg[lane + 64] : -1.0e300;
    double mx = fmax(p0, p1);
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
    p0 = lane < (int)experts ? exp(p0 - mx) : 0.0;
    p1 = lane + 64 < (int)experts ? exp(p1 - mx) : 0.0;
    const double den = wave_sum_d(p0 + p1);
    p0 /= den; p1 /= den;
    if (lane >= (int)experts) p0 = -2.0;
    if (lane + 64 >= (int)experts) p1 = -2.0;
    uint32_t ids[QXG_TOPK];
    double w[QXG_TOPK];
    for (int r = 0; r < QXG_TOPK; ++r) {
        // best by (p desc, index asc)
        double bp = p0; int bi = lane;
        if (p1 > bp) { bp = p1; bi = lane + 64; }
        for (int o = 32; o > 0; o >>= 1) {
            const double op = __shfl_xor(bp, o);
            const int oi = __shfl_xor(bi, o);
            if (op > bp || (op == bp && oi < bi)) { bp = op; bi = oi; }
        }
        ids[r] = bi < (int)experts ? (uint32_t)bi : 0u;   // never address past the expert array
        w[r] = bp;
        if (bi == lane) p0 = -2.0;
        if (bi == lane + 64) p1 = -2.0;
    }
    if (lane == 0) {
        double sel = 0.0;
        for (int r = 0; r < QXG_TOPK; ++r) sel += w[r];
        for (int r = 0; r < QXG_TOPK; ++r) { st->moe_ids[r] = ids[r]; st->moe_w[r] = w[r] / sel; }
        st->ctr_router = 0;
    }
}

// gate/up IQ2_XS (2048 -> 768, 8 selected experts) + SwiGLU
// h[r][i] = (float)(silu((double)g) * (double)u) (src/qx_format.c:5298, 2511-2513).
template <int UPW>
__global__ __launch_bounds__(256) void qxk_gate_up(const float *x, const float *norm_w,
        const uint8_t *g_qs, const uint8_t *g_sc, const uint16_t *g_d,
        const uint8_t *u_qs, const uint8_t *u_sc, const uint16_t *u_d,
        Tables T, const DevState *st, float *h) {
    __shared__ uint4 s_g2[512];
    __shared__ uint2 s_sel[128];
    load_g2(s_g2, s_sel, T);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 3, ib = lane & 7;
    Dig g;
    const bool ok = wave_all(norm_digits_2048(x, norm_w, lane, g));
    __syncthreads();
    const int u0 = (blockIdx.x * 4 + wave) * UPW;
    for (int uu = 0; uu < UPW; ++uu) {
        const int unit = u0 + uu;
        if (unit >= QXG_TOPK * QXG_FFN) break;
        const int r = unit / QXG_FFN, i = unit - r * QXG_FFN;
        const uint64_t blk = ((uint64_t)st->moe_ids[r] * QXG_FFN + i) * 8 + b;
        const uint2 gq = reinterpret_cast<const uint2 *>(g_qs + blk * 64)[ib];
        const uint2 uq = reinterpret_cast<const uint2 *>(u_qs + blk * 64)[ib];
        const float gs = wave_sum(dot_iq2(gq, g_sc[blk * 8 + ib], g_d[blk], g, s_g2, s_sel));
        const float us = wave_sum(dot_iq2(uq, u_sc[blk * 8 + ib], u_d[blk], g, s_g2, s_sel));
        if (lane == 0) {
            const float gv = (ok && isfinite(gs)) ? gs : 0.0f;
            const float uv = (ok && isfinite(us)) ? us : 0.0f;
            const double sg = (double)gv / (1.0 + exp(-(double)gv));
            h[unit] = (float)(sg * (double)uv);
        }
    }
}

// down IQ3_XXS (768 -> 2048) for the 8 experts, rank-ordered weighted f32 sum and
// residual: x[i] = x[i] + sum_r (float)(w_r * (double)y_r[i]) (src/qx_format.c:5296-5309).
// Wave per output row; lanes 8r..8r+7 hold rank r, lane 8r+k the sub-blocks k of blocks 0..2.
template <int RPW>
__global__ __launch_bounds__(256) void qxk_down(const float *h, const uint8_t *d_qs, const uint8_t *d_aux,
        const uint16_t *d_d, Tables T, const DevState *st, float *x, float *moe_dump) {
    __shared__ uint2 s_g3[256];
    __shared__ uint2 s_sel[128];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) s_g3[i] = T.g3[i];
    for (int i = threadIdx.x; i < 128; i += blockDim.x) s_sel[i] = T.sel[i];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane >> 3, k = lane & 7;
    const uint32_t e = st->moe_ids[r];
    Dig g[3];
    bool fin = true;
#pragma unroll
    for (int j = 0; j < 3; ++j) fin &= plain_digits(h + r * QXG_FFN + 256 * j + 32 * k, g[j]);
    const bool ok = wave_all(fin);
    __syncthreads();
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    for (int rr = 0; rr < RPW; ++rr) {
        const int row = r0 + rr;
        if (row >= 2048) break;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint64_t blk = ((uint64_t)e * 2048 + row) * 3 + j;
            const uint2 qv = reinterpret_cast<const uint2 *>(d_qs + blk * 64)[k];
            const uint32_t aux = reinterpret_cast<const uint32_t *>(d_aux + blk * 32)[k];
            part += dot_iq3(qv, aux, d_d[blk], g[j], s_g3, s_sel);
        }
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) part += __shfl_xor(part, o);
        const float y = (ok && isfinite(part)) ? part : 0.0f;
        float moe = 0.0f;
        for (int q = 0; q < QXG_TOPK; ++q) {
            const float yq = __shfl(y, 8 * q);
            moe += (float)(st->moe_w[q] * (double)yq);
        }
        if (lane == 0) {
            if (moe_dump) moe_dump[row] = moe;
            x[row] = x[row] + moe;
        }
    }
}

// output RMSNorm + Q6_K head (2048 -> vocab) -> f32 logits (src/qx_format.c:3554-3738).
// Skipped on prompt steps unless forced.  A non-finite logit sets st->nonfinite.
template <int RPW>
__global__ __launch_bounds__(256) void qxk_head(const float *x, const float *norm_w, const uint8_t *ql,
        const uint8_t *qh, const int8_t *sc, const uint16_t *dd, uint32_t vocab, DevState *st, float *logits,
        float *norm_dump) {
    if (!st->force_head && st->step + 1 < st->n_prompt) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 3, ib = lane & 7, hh = ib >> 2, k = ib & 3;
    Dig g;
    bool fin;
    {
        float v[32];
        const float4 *xp = reinterpret_cast<const float4 *>(x + 32 * lane);
        for (int i = 0; i < 8; ++i) { const float4 t = xp[i]; v[4*i] = t.x; v[4*i+1] = t.y; v[4*i+2] = t.z; v[4*i+3] = t.w; }
        double ss = 0.0;
        for (int i = 0; i < 32; ++i) ss += (double)v[i] * (double)v[i];
        ss = wave_sum_d(ss);
        const double rms = sqrt(ss / 2048.0 + 1.0e-6);
        for (int i = 0; i < 32; ++i) v[i] = (float)((double)v[i] / rms) * norm_w[32 * lane + i];
        if (norm_dump && blockIdx.x == 0 && wave == 0)
            for (int i = 0; i < 32; ++i) norm_dump[32 * lane + i] = v[i];
        fin = make_digits(v, g);
    }
    const bool ok = wave_all(fin);
    const Q6Bias bias = q6_bias(g);
    const uint32_t r0 = (blockIdx.x * 4 + wave) * RPW;
    for (int rr = 0; rr < RPW; ++rr) {
        const uint32_t r = r0 + rr;
        if (r >= vocab) break;
        const uint64_t blk = (uint64_t)r * 8 + b;
        const uint4 *lp = reinterpret_cast<const uint4 *>(ql + blk * 128 + 64 * hh + 32 * (k & 1));
        const uint4 *hp = reinterpret_cast<const uint4 *>(qh + blk * 64 + 32 * hh);
        const int8_t *sp = sc + blk * 16 + 8 * hh + 2 * k;
        const float s = wave_sum(dot_q6(lp[0], lp[1], hp[0], hp[1], sp[0], sp[1], dd[blk], ib, g, bias));
        if (lane == 0) {
            logits[r] = s;
            if (!ok || !isfinite(s)) st->nonfinite = 1u;
        }
    }
}

// top-N (N <= 32) over logits by (value desc, index asc): each block reduces a
// slice to N candidates, the last block merges; writes tokens[step+1] = argmax on
// generate steps.  Round r picks the best element strictly below pick r-1 in that
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
    if (!st->force_head && st->step + 1 < st->n_prompt) return;
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    __shared__ uint32_t ticket;
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
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) ticket = atomicAdd(&st->ctr_topk, 1u);
    __syncthreads();
    if (ticket != gridDim.x - 1) return;
    __threadfence();
    select_topn(cand_v, cand_i, gridDim.x * topn, topn, top_v, top_i, sv, si);
    if (threadIdx.x == 0) {
        st->ctr_topk = 0;
        if (st->step + 1 >= st->n_prompt) tokens[st->step + 1] = top_i[0];
    }
}

extern "C" __global__ void qxk_advance(DevState *st) {
    if (threadIdx.x == 0) st->step = st->step + 1;
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
    }
}

// ----------------------------------------------------------------- launch wrappers
extern "C" {
void qxl_qkv(hipStream_t s, const float *x, const float *nw, const QTensor *q, const QTensor *k, const QTensor *v, float *qkv) {
    constexpr int RPW = 4;
    hipLaunchKernelGGL(qxk_qkv<RPW>, dim3(5120 / (4 * RPW)), dim3(256), 0, s, x, nw, q->p0, q->p1, k->p0, k->p1, v->p0, v->p1, qkv);
}
void qxl_oproj(hipStream_t s, const float *ctxv, const QTensor *o, float *x, float *dump) {
    constexpr int RPW = 2;
    hipLaunchKernelGGL(qxk_oproj<RPW>, dim3(2048 / (4 * RPW)), dim3(256), 0, s, ctxv, o->p0, o->p1, x, dump);
}
void qxl_gate_up(hipStream_t s, const float *x, const float *nw, const QTensor *g, const QTensor *u, Tables T,
                 const DevState *st, float *h) {
    constexpr int UPW = 4;
    hipLaunchKernelGGL(qxk_gate_up<UPW>, dim3(QXG_TOPK * QXG_FFN / (4 * UPW)), dim3(256), 0, s, x, nw,
                       g->p0, g->p1, g->d, u->p0, u->p1, u->d, T, st, h);
}
void qxl_down(hipStream_t s, const float *h, const QTensor *d, Tables T, const DevState *st, float *x, float *dump) {
    constexpr int RPW = 2;
    hipLaunchKernelGGL(qxk_down<RPW>, dim3(2048 / (4 * RPW)), dim3(256), 0, s, h, d->p0, d->p1, d->d, T, st, x, dump);
}
void qxl_head(hipStream_t s, const float *x, const float *nw, const QTensor *w, uint32_t vocab, DevState *st,
              float *logits, float *norm_dump) {
    constexpr int RPW = 8;
    const uint32_t grid = (vocab + 4 * RPW - 1) / (4 * RPW);
    hipLaunchKernelGGL(qxk_head<RPW>, dim3(grid), dim3(256), 0, s, x, nw, w->p0, w->p1, (const int8_t *)w->p2, w->d,
                       vocab, st, logits, norm_dump);
}
}
