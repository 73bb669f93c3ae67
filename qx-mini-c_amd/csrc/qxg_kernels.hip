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

DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// ---- DPP lane exchanges (VALU latency; __shfl_xor lowers to ds_bpermute through LDS).
// quad_perm xor1 = [1,0,3,2], xor2 = [2,3,0,1]; row_ror:4/8 rotate within a 16-lane
// row; row_half_mirror pairs lane i with 7-i inside each group of 8.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128, DPP_HALF_MIRROR = 0x141 };

template <int CTRL>
DEV float dppf(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false)); }
template <int CTRL>
DEV int dppi(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
DEV double dppd(double v) {
    const int2 h = *reinterpret_cast<int2 *>(&v);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(0, h.x, CTRL, 0xf, 0xf, false);
    r.y = __builtin_amdgcn_update_dpp(0, h.y, CTRL, 0xf, 0xf, false);
    return *reinterpret_cast<double *>(&r);
}
DEV float rdlanef(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
DEV double rdlaned(double v, int l) {
    const int2 h = *reinterpret_cast<int2 *>(&v);
    int2 r;
    r.x = __builtin_amdgcn_readlane(h.x, l);
    r.y = __builtin_amdgcn_readlane(h.y, l);
    return *reinterpret_cast<double *>(&r);
}
// sum over each 16-lane row, result in every lane of the row
DEV double row16_sum_d(double v) {
    v += dppd<DPP_XOR1>(v); v += dppd<DPP_XOR2>(v); v += dppd<DPP_ROR4>(v); v += dppd<DPP_ROR8>(v);
    return v;
}
// wave totals, uniform (rows combined in lane order 0, 16, 32, 48)
DEV double wave_total_d(double v) {
    v = row16_sum_d(v);
    return (rdlaned(v, 0) + rdlaned(v, 16)) + (rdlaned(v, 32) + rdlaned(v, 48));
}
DEV double wave_max_d(double v) {
    v = fmax(v, dppd<DPP_XOR1>(v)); v = fmax(v, dppd<DPP_XOR2>(v));
    v = fmax(v, dppd<DPP_ROR4>(v)); v = fmax(v, dppd<DPP_ROR8>(v));
    return fmax(fmax(rdlaned(v, 0), rdlaned(v, 16)), fmax(rdlaned(v, 32), rdlaned(v, 48)));
}

// 32 activations of one group as three int8 digit planes and a power-of-two scale
struct Dig {
    uint32_t h[8], m[8], l[8];
    float s;
};

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
DEV void load32(const float *p, float *v) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

// reference qx_apply_f32_rmsnorm (src/qx_format.c:3358-3371): double sum of
// squares, rms = sqrt(ss/n + 1e-6), y = (float)(x/rms) * w.  The lane holds the
// 32 values [32*lane, 32*lane+32) of a 2048-vector (already loaded); the wave
// reduces.  x/rms is formed as x*(1/rms) in double; after the cast to f32 the two
// differ only when x/rms lies within 2^-53 relative of an f32 rounding boundary.
DEV void rmsnorm32(float *v, const float *w) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 32; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_total_d(ss);
    const double inv = 1.0 / sqrt(ss / 2048.0 + 1.0e-6);
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = (float)((double)v[i] * inv) * w[i];
}


// ---- block-cooperative activation digits.  The digit planes of all N/32 groups of
// a vector are computed once per block into LDS (DIG_STRIDE dwords per group: h[8],
// m[8], l[8], scale bits), 8 consecutive values per thread; the 4 threads of a group
// form a quad, so the group max is two in-quad DPP exchanges.  With NORM, the vector
// is first RMS-normalised with weights w (reference src/qx_format.c:3358-3371).
constexpr int DIG_STRIDE = 28;   // 16-byte aligned rows for ds_read_b128

DEV void digits8(const float *y, float mx, uint32_t &ph0, uint32_t &ph1, uint32_t &pm0, uint32_t &pm1, uint32_t &pl0,
                 uint32_t &pl1, float &scale) {
    int e = 0;
    if (mx > 0.0f) (void)frexpf(mx, &e);
    scale = mx > 0.0f ? ldexpf(1.0f, e - 22) : 0.0f;
    uint32_t H[2] = {0, 0}, M[2] = {0, 0}, L[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int X = mx > 0.0f ? (int)rintf(ldexpf(y[i], 22 - e)) : 0;
        const int l = ((X + 128) & 255) - 128;
        const int X1 = (X - l) >> 8;
        const int m = ((X1 + 128) & 255) - 128;
        const int hh = (X1 - m) >> 8;
        H[i >> 2] |= (uint32_t)(hh & 255) << (8 * (i & 3));
        M[i >> 2] |= (uint32_t)(m & 255) << (8 * (i & 3));
        L[i >> 2] |= (uint32_t)(l & 255) << (8 * (i & 3));
    }
    ph0 = H[0]; ph1 = H[1]; pm0 = M[0]; pm1 = M[1]; pl0 = L[0]; pl1 = L[1];
}

// The vector (and norm weights) as loaded by one thread: 8 consecutive values per
// chunk.  Kernels issue these loads before their weight loads, so the activation
// arrives first and the digit work overlaps the weight fetch.
template <int N, bool NORM>
struct DigIn {
    static constexpr int NCH = N / 8, PER = (NCH + 255) / 256;
    float v[PER][8];
    float w[NORM ? 8 : 1];
};

template <int N, bool NORM>
DEV void digits_load(const float *x, const float *w, DigIn<N, NORM> &in) {
    using D = DigIn<N, NORM>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < D::PER; ++it) {
        const int c = tid + 256 * it;
        if (c < D::NCH) {
            const float4 a = reinterpret_cast<const float4 *>(x)[2 * c], b = reinterpret_cast<const float4 *>(x)[2 * c + 1];
            in.v[it][0] = a.x; in.v[it][1] = a.y; in.v[it][2] = a.z; in.v[it][3] = a.w;
            in.v[it][4] = b.x; in.v[it][5] = b.y; in.v[it][6] = b.z; in.v[it][7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) in.v[it][i] = 0.0f;
        }
    }
    if constexpr (NORM) {
        static_assert(D::PER == 1, "normalised vectors are 2048 long");
        const float4 a = reinterpret_cast<const float4 *>(w)[2 * tid], b = reinterpret_cast<const float4 *>(w)[2 * tid + 1];
        in.w[0] = a.x; in.w[1] = a.y; in.w[2] = a.z; in.w[3] = a.w;
        in.w[4] = b.x; in.w[5] = b.y; in.w[6] = b.z; in.w[7] = b.w;
    }
}

// returns true when every value is finite (block-uniform); ends with a block barrier
template <int N, bool NORM>
DEV bool block_digits(DigIn<N, NORM> &in, uint32_t *s_dig, double *s_red, float *norm_out = nullptr) {
    using D = DigIn<N, NORM>;
    const int tid = threadIdx.x;
    if constexpr (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (double)in.v[0][i] * (double)in.v[0][i];
        ss = wave_total_d(ss);
        if ((tid & 63) == 0) s_red[tid >> 6] = ss;
        __syncthreads();
        const double tot = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
        const double inv = 1.0 / sqrt(tot / (double)N + 1.0e-6);
#pragma unroll
        for (int i = 0; i < 8; ++i) in.v[0][i] = (float)((double)in.v[0][i] * inv) * in.w[i];
        if (norm_out) {
            reinterpret_cast<float4 *>(norm_out)[2 * tid] = make_float4(in.v[0][0], in.v[0][1], in.v[0][2], in.v[0][3]);
            reinterpret_cast<float4 *>(norm_out)[2 * tid + 1] = make_float4(in.v[0][4], in.v[0][5], in.v[0][6], in.v[0][7]);
        }
    }
    bool fin = true;
#pragma unroll
    for (int it = 0; it < D::PER; ++it) {
        const int c = tid + 256 * it;
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) { fin = fin && isfinite(in.v[it][i]); mx = fmaxf(mx, fabsf(in.v[it][i])); }
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
        if (c < D::NCH) {
            uint32_t h0, h1, m0, m1, l0, l1;
            float sc;
            digits8(in.v[it], isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
            uint32_t *d = s_dig + (c >> 2) * DIG_STRIDE;
            const int q = c & 3;
            *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
            *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
            *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
            if (q == 0) d[24] = __float_as_uint(sc);
        }
    }
    return __syncthreads_or(!fin) == 0;
}

DEV void load_dig(const uint32_t *__restrict__ s_dig, int g, Dig &d) {
    const uint4 *p = reinterpret_cast<const uint4 *>(s_dig + g * DIG_STRIDE);
    const uint4 a = p[0], b = p[1], c = p[2], e = p[3], f = p[4], k = p[5];
    d.h[0] = a.x; d.h[1] = a.y; d.h[2] = a.z; d.h[3] = a.w; d.h[4] = b.x; d.h[5] = b.y; d.h[6] = b.z; d.h[7] = b.w;
    d.m[0] = c.x; d.m[1] = c.y; d.m[2] = c.z; d.m[3] = c.w; d.m[4] = e.x; d.m[5] = e.y; d.m[6] = e.z; d.m[7] = e.w;
    d.l[0] = f.x; d.l[1] = f.y; d.l[2] = f.z; d.l[3] = f.w; d.l[4] = k.x; d.l[5] = k.y; d.l[6] = k.z; d.l[7] = k.w;
    d.s = __uint_as_float(s_dig[g * DIG_STRIDE + 24]);
}


DEV uint32_t cur_pos(const DevState *st) { return st->pos0 + st->step; }

// R per-lane partial sums (one per row, R in {1,2,4,8}) reduced over the wave:
// up to two split rounds inside each quad (a lane keeps half of the rows and adds
// its partner's half), then row16 sums, then the four rows of the wave through
// readlane.  out[r] is the total of row r, wave-uniform.
template <int R>
DEV void rows_reduce(float (&v)[R], float (&out)[R], int lane) {
    constexpr int S = R >= 4 ? 2 : (R == 2 ? 1 : 0);   // quad split rounds
    constexpr int K = R >> S;                          // values left per lane
    const bool b0 = lane & 1, b1 = (lane >> 1) & 1;
    if constexpr (S >= 1) {
        constexpr int half = R / 2;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float send = b0 ? v[i] : v[half + i];
            const float keep = b0 ? v[half + i] : v[i];
            v[i] = keep + dppf<DPP_XOR1>(send);
        }
    }
    if constexpr (S >= 2) {
        constexpr int half = R / 4;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float send = b1 ? v[i] : v[half + i];
            const float keep = b1 ? v[half + i] : v[i];
            v[i] = keep + dppf<DPP_XOR2>(send);
        }
    }
#pragma unroll
    for (int i = 0; i < K; ++i) {
        if constexpr (S == 0) { v[i] += dppf<DPP_XOR1>(v[i]); }
        if constexpr (S <= 1) { v[i] += dppf<DPP_XOR2>(v[i]); }
        v[i] += dppf<DPP_ROR4>(v[i]);
        v[i] += dppf<DPP_ROR8>(v[i]);
    }
    // lane L (low bits b0,b1) holds rows base..base+K-1 with base = K*(2^(S-1)*b0 + ...)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int l0, j;
        if constexpr (S == 0) { l0 = 0; j = r; }
        else if constexpr (S == 1) { l0 = r / K; j = r % K; }               // b0 = subset
        else { const int sub = r / K; l0 = (sub >> 1) | ((sub & 1) << 1); j = r % K; }  // subset = 2*b0 + b1
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < K; ++i) if (i == j) t = v[i];
        out[r] = (rdlanef(t, l0) + rdlanef(t, l0 + 16)) + (rdlanef(t, l0 + 32) + rdlanef(t, l0 + 48));
    }
}

}  // namespace

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
// Wave per RPW consecutive rows; lane = 8*block + sub-block.  Every global load of
// the wave is issued before the norm/digit prologue so their latencies overlap.
template <int RPW>
__global__ __launch_bounds__(256) void qxk_qkv(const float *x, const float *norm_w,
        const uint8_t *q_qs, const uint8_t *q_meta, const uint8_t *k_qs, const uint8_t *k_meta,
        const uint8_t *v_qs, const uint8_t *v_meta, float *qkv) {
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 3, ib = lane & 7;
    const int r0 = (blockIdx.x * 4 + wave) * RPW;   // grid covers exactly 5120 rows
    QXG_MARK(3, 0);
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    uint4 qv[RPW];
    uint2 mv[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const int r = r0 + rr;
        const uint8_t *qs, *meta;
        int lr;
        if (r < 4096) { qs = q_qs; meta = q_meta; lr = r; }
        else if (r < 4608) { qs = k_qs; meta = k_meta; lr = r - 4096; }
        else { qs = v_qs; meta = v_meta; lr = r - 4608; }
        const uint64_t blk = (uint64_t)lr * 8 + b;
        qv[rr] = reinterpret_cast<const uint4 *>(qs + blk * 128)[ib];
        mv[rr] = *reinterpret_cast<const uint2 *>(meta + blk * 8);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_ANCHOR(din.v[0][7]);
    QXG_MARK(3, 1);
    const bool ok = block_digits(din, s_dig, s_red);
    QXG_MARK(3, 2);
    Dig g;
    load_dig(s_dig, lane, g);
    float part[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) part[rr] = dot_iq4(qv[rr], mv[rr], ib, g);
    QXG_ANCHOR(part[0]); QXG_ANCHOR(part[RPW - 1]);
    QXG_MARK(3, 3);
    float out[RPW];
    rows_reduce<RPW>(part, out, lane);
    float mine = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) if (lane == rr) mine = out[rr];
    if (lane < RPW) qkv[r0 + lane] = (ok && isfinite(mine)) ? mine : 0.0f;
    QXG_MARK(3, 4);
}

// Attention for one q head, with the per-head q/k RMSNorm (src/qx_format.c:3740-3757),
// split-half RoPE (4625-4641; cos/sin from the host-computed table) and INT8 K/V
// quantization (4449-4463) of the current position fused in: every block derives the
// same K/V row (the scale spans all 512 values), block 0 stores it at [layer][pos],
// and each block uses its own copy for position pos.  Scores (double) over 0..pos,
// double softmax, f32 context accumulation per position in position order within
// each of two position halves (reference src/qx_format.c:5127-5172).
// The cached K/V rows of positions [0, min(pos, ATT_STAGE)) and their scales are
// loaded at kernel start, together with q/k/v, and staged in LDS while the norm,
// RoPE and quantization run; later positions are read from global memory.
namespace {
DEV float block_max256(float v, float *red) {
    v = fmaxf(v, dppf<DPP_XOR1>(v)); v = fmaxf(v, dppf<DPP_XOR2>(v));
    v = fmaxf(v, dppf<DPP_ROR4>(v)); v = fmaxf(v, dppf<DPP_ROR8>(v));
    v = fmaxf(fmaxf(rdlanef(v, 0), rdlanef(v, 16)), fmaxf(rdlanef(v, 32), rdlanef(v, 48)));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// 128 values of one head held as (lane, lane+64) by a wave: per-head RMSNorm then RoPE
DEV void head_norm_rope_wave(float &x0, float &x1, float w0, float w1, double c, double s) {
    const double ss = wave_total_d((double)x0 * (double)x0 + (double)x1 * (double)x1);
    const double inv = 1.0 / sqrt(ss / 128.0 + 1.0e-6);
    const float n0 = (float)((double)x0 * inv * (double)w0);
    const float n1 = (float)((double)x1 * inv * (double)w1);
    x0 = (float)((double)n0 * c - (double)n1 * s);
    x1 = (float)((double)n0 * s + (double)n1 * c);
}
}  // namespace

constexpr int ATT_STAGE = 128;   // positions staged in LDS (4 uint4 of K and of V per thread)

extern "C" __global__ __launch_bounds__(256) void qxk_attn(const float *qkv, const float *q_norm, const float *k_norm,
        Tables T, int8_t *kc, int8_t *vc, float *ks, float *vs, uint32_t layer, uint32_t ctx, double sqrt_hd,
        const DevState *st, float *ctx_out, float *vcur_dump) {
    extern __shared__ double s_sc[];               // ctx scores
    __shared__ uint4 s_kst[ATT_STAGE * 8], s_vst[ATT_STAGE * 8];   // staged rows of this kv head
    __shared__ float s_kss[ATT_STAGE], s_vss[ATT_STAGE];
    __shared__ float s_k[512], s_v[512];
    __shared__ double s_q[128];
    __shared__ float red[4];
    __shared__ float s_part[2][128];
    __shared__ int8_t s_k8[128], s_v8[128];
    __shared__ float s_scale[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qh = blockIdx.x, kvh = qh >> 3;
    const uint32_t pos = cur_pos(st), n = pos + 1;
    const uint64_t base = (uint64_t)layer * ctx;
    const uint32_t nst = pos < (uint32_t)ATT_STAGE ? pos : (uint32_t)ATT_STAGE;   // staged positions
    // cached rows first: 16 bytes of row (tid>>3) + 32*i, chunk tid&7, i < 4
    uint4 kst[4], vst[4];
    float kss = 0.0f, vss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        if (t < nst) {
            const uint64_t off = (base + t) * 512 + kvh * 128 + 16 * (tid & 7);
            kst[i] = *reinterpret_cast<const uint4 *>(kc + off);
            vst[i] = *reinterpret_cast<const uint4 *>(vc + off);
        }
    }
    if ((uint32_t)tid < nst) { kss = ks[base + tid]; vss = vs[base + tid]; }
    // loads: k head `wave`, v (2 per thread), q head (wave 0 after k), norms, rope row
    float k0 = qkv[4096 + 128 * wave + lane], k1 = qkv[4096 + 128 * wave + 64 + lane];
    const float v0 = qkv[4608 + tid], v1 = qkv[4608 + 256 + tid];
    float q0 = qkv[128 * qh + lane], q1 = qkv[128 * qh + 64 + lane];
    const float kw0 = k_norm[lane], kw1 = k_norm[64 + lane], qw0 = q_norm[lane], qw1 = q_norm[64 + lane];
    const double c = T.rope_cos[pos * 64 + lane], s = T.rope_sin[pos * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    head_norm_rope_wave(k0, k1, kw0, kw1, c, s);
    s_k[128 * wave + lane] = k0;
    s_k[128 * wave + 64 + lane] = k1;
    s_v[tid] = v0;
    s_v[256 + tid] = v1;
    if (wave == 0) {
        head_norm_rope_wave(q0, q1, qw0, qw1, c, s);
        s_q[lane] = (double)q0;
        s_q[64 + lane] = (double)q1;
    }
    // INT8 quantize K and V over all 512 values (scale = max|x|/127, 1 if zero)
    float ka = 0.0f, va = 0.0f;
    {
        const float a0 = isfinite(k0) ? fabsf(k0) : 0.0f, a1 = isfinite(k1) ? fabsf(k1) : 0.0f;
        ka = fmaxf(a0, a1);
        const float b0 = isfinite(v0) ? fabsf(v0) : 0.0f, b1 = isfinite(v1) ? fabsf(v1) : 0.0f;
        va = fmaxf(b0, b1);
    }
    ka = block_max256(ka, red);
    va = block_max256(va, red);
    const float kscale = ka > 0.0f ? ka / 127.0f : 1.0f, vscale = va > 0.0f ? va / 127.0f : 1.0f;
    const uint64_t slot = base + pos;
    for (int i = tid; i < 512; i += 256) {
        const float kx = s_k[i], vx = s_v[i];
        int qk = isfinite(kx) ? (int)rintf(kx / kscale) : 0;
        int qv = isfinite(vx) ? (int)rintf(vx / vscale) : 0;
        qk = qk < -127 ? -127 : qk > 127 ? 127 : qk;
        qv = qv < -127 ? -127 : qv > 127 ? 127 : qv;
        if (blockIdx.x == 0) { kc[slot * 512 + i] = (int8_t)qk; vc[slot * 512 + i] = (int8_t)qv; }
        if ((i >> 7) == kvh) { s_k8[i & 127] = (int8_t)qk; s_v8[i & 127] = (int8_t)qv; }
    }
    if (blockIdx.x == 0 && tid == 0) { ks[slot] = kscale; vs[slot] = vscale; }
    if (blockIdx.x == 0 && vcur_dump) { vcur_dump[tid] = v0; vcur_dump[256 + tid] = v1; }
    if (tid == 0) { s_scale[0] = kscale; s_scale[1] = vscale; }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (tid >> 3) + 32 * i;
        if (t < nst) { s_kst[t * 8 + (tid & 7)] = kst[i]; s_vst[t * 8 + (tid & 7)] = vst[i]; }
    }
    if ((uint32_t)tid < nst) { s_kss[tid] = kss; s_vss[tid] = vss; }
    __syncthreads();
    // scores: 16 lanes per position, 8 dims per lane
    {
        const int sub = lane >> 4, dl = lane & 15;
        double qd[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qd[j] = s_q[8 * dl + j];
        for (uint32_t t0 = 4 * wave; t0 < n; t0 += 16) {
            const uint32_t t = t0 + sub;
            double acc = 0.0;
            if (t < n) {
                uint2 kk;
                float ksc;
                if (t == pos) {
                    kk = *reinterpret_cast<const uint2 *>(s_k8 + 8 * dl);
                    ksc = s_scale[0];
                } else if (t < nst) {
                    kk = reinterpret_cast<const uint2 *>(s_kst)[t * 16 + dl];
                    ksc = s_kss[t];
                } else {
                    kk = *reinterpret_cast<const uint2 *>(kc + (base + t) * 512 + kvh * 128 + 8 * dl);
                    ksc = ks[base + t];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int8_t kb = (int8_t)(((j < 4 ? kk.x : kk.y) >> (8 * (j & 3))) & 255u);
                    acc += qd[j] * (double)((float)kb * ksc);
                }
            }
            acc = row16_sum_d(acc);   // 16 lanes = one position
            if (t < n && dl == 0) {
                double sc = acc / sqrt_hd;
                if (!isfinite(sc)) sc = 0.0;
                s_sc[t] = sc;
            }
        }
    }
    __syncthreads();
    // softmax in double
    double mx = -1.0e300;
    for (uint32_t t = tid; t < n; t += 256) mx = fmax(mx, s_sc[t]);
    mx = wave_max_d(mx);
    __shared__ double redd[4];
    if (lane == 0) redd[wave] = mx;
    __syncthreads();
    mx = fmax(fmax(redd[0], redd[1]), fmax(redd[2], redd[3]));
    double den = 0.0;
    for (uint32_t t = tid; t < n; t += 256) {
        const double e = exp(s_sc[t] - mx);
        s_sc[t] = e;
        den += e;
    }
    den = wave_total_d(den);
    __syncthreads();
    if (lane == 0) redd[wave] = den;
    __syncthreads();
    den = (redd[0] + redd[1]) + (redd[2] + redd[3]);
    if (!isfinite(den) || den <= 0.0) den = 1.0;
    // context: thread (d, half); positions of each half in order
    const int d = tid & 127, hf = tid >> 7;
    const uint32_t t0 = hf ? n / 2 : 0, t1 = hf ? n : n / 2;
    float acc = 0.0f;
    for (uint32_t t = t0; t < t1; ++t) {
        const double wgt = s_sc[t] / den;
        const float vv = t == pos ? (float)s_v8[d] * s_scale[1]
                         : t < nst ? (float)reinterpret_cast<const int8_t *>(s_vst)[t * 128 + d] * s_vss[t]
                                   : (float)vc[(base + t) * 512 + kvh * 128 + d] * vs[base + t];
        acc += (float)(wgt * (double)vv);
    }
    s_part[hf][d] = acc;
    __syncthreads();
    if (tid < 128) ctx_out[qh * 128 + tid] = s_part[0][tid] + s_part[1][tid];
}

// O projection IQ4_XS 4096 -> 2048 on ctx, then x[r] += o[r] (src/qx_format.c:6420-6423).
// Lane handles sub-blocks lane and lane+64 (blocks lane/8 and 8+lane/8).
template <int RPW>
__global__ __launch_bounds__(256) void qxk_oproj(const float *ctxv, const uint8_t *qs, const uint8_t *meta,
                                                  float *x, float *attn_dump) {
    __shared__ uint32_t s_dig[128 * DIG_STRIDE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ib = lane & 7, b0 = lane >> 3, b1 = 8 + (lane >> 3);
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    QXG_MARK(0, 0);
    DigIn<4096, false> din;
    digits_load(ctxv, nullptr, din);
    const float xr = lane < RPW ? x[r0 + lane] : 0.0f;
    uint4 q0[RPW], q1[RPW];
    uint2 m0[RPW], m1[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const uint64_t k0 = (uint64_t)(r0 + rr) * 16 + b0, k1 = (uint64_t)(r0 + rr) * 16 + b1;
        q0[rr] = reinterpret_cast<const uint4 *>(qs + k0 * 128)[ib];
        q1[rr] = reinterpret_cast<const uint4 *>(qs + k1 * 128)[ib];
        m0[rr] = *reinterpret_cast<const uint2 *>(meta + k0 * 8);
        m1[rr] = *reinterpret_cast<const uint2 *>(meta + k1 * 8);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_ANCHOR(din.v[1][7]);
    QXG_MARK(0, 1);
    const bool ok = block_digits(din, s_dig, nullptr);
    QXG_MARK(0, 2);
    Dig g0, g1;
    load_dig(s_dig, lane, g0);
    load_dig(s_dig, lane + 64, g1);
    float part[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) part[rr] = dot_iq4(q0[rr], m0[rr], ib, g0) + dot_iq4(q1[rr], m1[rr], ib, g1);
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
    QXG_MARK(0, 4);
}

// ffn RMSNorm + F32 router logits in double (reference src/qx_format.c:5254-5264);
// wave per expert row.  The softmax and top-8 run in the prologue of the gate/up
// kernel, where the expert ids are needed.
extern "C" __global__ __launch_bounds__(256) void qxk_router(const float *x, const float *norm_w, const float *router,
        uint32_t experts, double *logits) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t e = blockIdx.x * 4 + wave;
    if (e >= experts) return;
    float v[32], w[32], r[32];
    load32(router + (uint64_t)e * 2048 + 32 * lane, r);
    load32(x + 32 * lane, v);
    load32(norm_w + 32 * lane, w);
    rmsnorm32(v, w);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 32; ++i) acc += (double)r[i] * (double)v[i];
    acc = wave_total_d(acc);
    if (lane == 0) logits[e] = acc;
}

namespace {
// order-preserving int32 image of a float (NaN sorts below everything)
DEV int order_key(double v) {
    if (v != v) return INT_MIN;
    const int b = __float_as_int((float)v);
    return b ^ ((b >> 31) & 0x7fffffff);
}
DEV int wave_max_i(int v) {
    v = max(v, dppi<DPP_XOR1>(v)); v = max(v, dppi<DPP_XOR2>(v));
    v = max(v, dppi<DPP_ROR4>(v)); v = max(v, dppi<DPP_ROR8>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Router top-8 and renormalised weights (src/qx_format.c:5265-5285), by every wave of
// the expert kernel on its own (no block barrier).  Lane l holds the logits of experts
// l and l+64 (double).  The reference picks by softmax probability with repeated
// strict-> scans (larger first, lower index on ties); the probability is a
// non-decreasing function of the logit, so picking by logit gives the same experts
// except where two probabilities round to the same double (a zero margin).  Each round
// takes the largest f32 key (float rounding is monotone); when several experts share
// that key the doubles decide, lower index on ties.  The weights p_r / sum_q p_q equal
// e_r / sum_q e_q with e = exp(l - l_max), since the softmax denominator cancels.
// ids[r] and w[r] are wave-uniform.
DEV void wave_top8(double l0, double l1, int E, uint32_t (&ids)[QXG_TOPK], double (&w)[QXG_TOPK]) {
    const int lane = threadIdx.x & 63;
    int k0 = lane < E ? order_key(l0) : INT_MIN, k1 = lane + 64 < E ? order_key(l1) : INT_MIN;
#pragma unroll
    for (int r = 0; r < QXG_TOPK; ++r) {
        const int m = wave_max_i(max(k0, k1));
        const uint64_t b0 = __ballot(k0 == m), b1 = __ballot(k1 == m);
        uint32_t id = 0;
        if (m == INT_MIN) {
            id = 0;                                  // nothing left (non-finite logits)
        } else if (__popcll(b0) + __popcll(b1) == 1) {
            id = b0 ? (uint32_t)__builtin_ctzll(b0) : 64u + (uint32_t)__builtin_ctzll(b1);
        } else {                                     // equal f32 keys: compare the doubles
            double best = 0.0;
            bool found = false;
            for (uint64_t b = b0; b; b &= b - 1) {
                const int j = __builtin_ctzll(b);
                const double v = rdlaned(l0, j);
                if (!found || v > best) { best = v; id = (uint32_t)j; found = true; }
            }
            for (uint64_t b = b1; b; b &= b - 1) {
                const int j = __builtin_ctzll(b);
                const double v = rdlaned(l1, j);
                if (!found || v > best) { best = v; id = 64u + (uint32_t)j; found = true; }
            }
        }
        ids[r] = id;
        if (m != INT_MIN && lane == (int)(id & 63u)) {
            if (id < 64u) k0 = INT_MIN; else k1 = INT_MIN;
        }
    }
    // lane q < 8 takes the logit of pick q; e_q = exp(l_q - l_0), l_0 the largest
    double lq = 0.0;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) {
        const double v = ids[q] < 64u ? rdlaned(l0, (int)ids[q]) : rdlaned(l1, (int)(ids[q] - 64u));
        if (lane == q) lq = v;
    }
    const double lmax = rdlaned(lq, 0);
    const double eq = lane < QXG_TOPK ? exp(lq - lmax) : 0.0;
    double sel = 0.0;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) sel += rdlaned(eq, q);   // rank order, as the reference
    const double wq = eq / sel;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) w[q] = rdlaned(wq, q);
}
}  // namespace

// gate/up IQ2_XS (2048 -> 768) for the 8 routed experts (ids from st) + SwiGLU
// h[r][i] = (float)(silu((double)g) * (double)u) (src/qx_format.c:5298, 2511-2513).
// Weight loads are issued first; the codebook tables go to LDS while they fly.
// Units are processed in a rolled loop whose prefetch registers shift by one unit per
// iteration (static indices keep them in VGPRs).
template <int UPW>
__global__ __launch_bounds__(256) void qxk_gate_up(const float *x, const float *norm_w,
        const uint8_t *g_qs, const uint8_t *g_sc, const uint16_t *g_d,
        const uint8_t *u_qs, const uint8_t *u_sc, const uint16_t *u_d, Tables T, const double *logits,
        uint32_t experts, DevState *st, float *h) {
    __shared__ uint4 s_g2[512];
    __shared__ uint2 s_sel[128];
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = lane >> 3, ib = lane & 7;
    const int u0 = (blockIdx.x * 4 + wave) * UPW;   // grid covers exactly 8*768 units
    const int E = (int)experts;
    QXG_MARK(1, 0);
    // the router logits head the longest chain (logits -> top-8 -> weights): loaded first
    const double l0 = lane < E ? logits[lane] : 0.0, l1 = lane + 64 < E ? logits[lane + 64] : 0.0;
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    const uint4 t0 = T.g2[tid], t1 = T.g2[tid + 256];
    const uint2 t2 = T.sel[tid & 127];
    QXG_ANCHOR(l1);
    QXG_MARK(1, 5);
    uint32_t ids[QXG_TOPK];
    double wts[QXG_TOPK];
    wave_top8(l0, l1, E, ids, wts);
    QXG_MARK(1, 6);
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) ids[q] = ids[q] < experts ? ids[q] : 0u;   // never address past the experts
    if (blockIdx.x == 0 && wave == 0) {   // the down kernel reads ids and renormalised weights from st
#pragma unroll
        for (int q = 0; q < QXG_TOPK; ++q)
            if (lane == q) { st->moe_ids[q] = ids[q]; st->moe_w[q] = wts[q]; }
    }
    uint32_t e = ids[0];
#pragma unroll
    for (int q = 1; q < QXG_TOPK; ++q) if (u0 / QXG_FFN == q) e = ids[q];   // 4 | 768: one expert per wave
    e = __builtin_amdgcn_readfirstlane(e);
    uint2 gq[UPW], uq[UPW];
    uint32_t gs[UPW], us[UPW], gd[UPW], ud[UPW];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
        const int i = (u0 + uu) % QXG_FFN;
        const uint64_t blk = ((uint64_t)e * QXG_FFN + i) * 8 + b;
        gq[uu] = reinterpret_cast<const uint2 *>(g_qs + blk * 64)[ib];
        uq[uu] = reinterpret_cast<const uint2 *>(u_qs + blk * 64)[ib];
        gs[uu] = g_sc[blk * 8 + ib];
        us[uu] = u_sc[blk * 8 + ib];
        gd[uu] = g_d[blk];
        ud[uu] = u_d[blk];
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    QXG_MARK(1, 7);
    s_g2[tid] = t0;
    s_g2[tid + 256] = t1;
    if (tid < 128) s_sel[tid] = t2;
    QXG_ANCHOR(din.v[0][7]);
    QXG_MARK(1, 1);
    const bool ok = block_digits(din, s_dig, s_red);   // ends with a barrier
    QXG_MARK(1, 2);
    Dig g;
    load_dig(s_dig, lane, g);
    // dots unit by unit in a rolled loop (prefetch registers and results shift by one
    // slot per iteration, so every index is static), then one reduction for all units
    float pg[UPW], pu[UPW];
#pragma unroll 1
    for (int uu = 0; uu < UPW; ++uu) {
        const float a = dot_iq2(gq[0], gs[0], gd[0], g, s_g2, s_sel);
        const float c = dot_iq2(uq[0], us[0], ud[0], g, s_g2, s_sel);
#pragma unroll
        for (int k = 0; k + 1 < UPW; ++k) {
            gq[k] = gq[k + 1]; uq[k] = uq[k + 1]; gs[k] = gs[k + 1]; us[k] = us[k + 1]; gd[k] = gd[k + 1]; ud[k] = ud[k + 1];
            pg[k] = pg[k + 1]; pu[k] = pu[k + 1];
        }
        pg[UPW - 1] = a;
        pu[UPW - 1] = c;
    }
    QXG_ANCHOR(pg[0]);
    QXG_MARK(1, 3);
    float p[2 * UPW], o[2 * UPW];
#pragma unroll
    for (int k = 0; k < UPW; ++k) { p[k] = pg[k]; p[UPW + k] = pu[k]; }
    rows_reduce<2 * UPW>(p, o, lane);
    float gv = 0.0f, uv = 0.0f;
#pragma unroll
    for (int k = 0; k < UPW; ++k) if (lane == k) { gv = o[k]; uv = o[UPW + k]; }
    if (lane < UPW) {
        gv = (ok && isfinite(gv)) ? gv : 0.0f;
        uv = (ok && isfinite(uv)) ? uv : 0.0f;
        const double sg = (double)gv / (1.0 + exp(-(double)gv));
        h[u0 + lane] = (float)(sg * (double)uv);
    }
    QXG_MARK(1, 4);
}

// down IQ3_XXS (768 -> 2048) for the 8 experts, rank-ordered weighted f32 sum and
// residual: x[i] = x[i] + sum_r (float)(w_r * (double)y_r[i]) (src/qx_format.c:5296-5309).
// Wave per output row; lanes 8r..8r+7 hold rank r, lane 8r+k the sub-blocks k of blocks 0..2.
template <int RPW>
__global__ __launch_bounds__(256) void qxk_down(const float *h, const uint8_t *d_qs, const uint8_t *d_aux,
        const uint16_t *d_d, Tables T, const DevState *st, float *x, float *moe_dump) {
    __shared__ uint2 s_g3[256];
    __shared__ uint2 s_sel[128];
    __shared__ uint32_t s_dig[192 * DIG_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    const uint2 t0 = T.g3[tid], t1 = T.sel[tid & 127];
    uint2 qv[RPW][3];
    uint32_t aux[RPW][3], dd[RPW][3];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint64_t blk = ((uint64_t)e * 2048 + r0 + rr) * 3 + j;
            qv[rr][j] = reinterpret_cast<const uint2 *>(d_qs + blk * 64)[k];
            aux[rr][j] = reinterpret_cast<const uint32_t *>(d_aux + blk * 32)[k];
            dd[rr][j] = d_d[blk];
        }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the first use
    s_g3[tid] = t0;
    if (tid < 128) s_sel[tid] = t1;
    QXG_ANCHOR(din.v[din.PER - 1][7]);
    QXG_MARK(2, 1);
    const bool ok = block_digits(din, s_dig, nullptr);   // ends with a barrier
    QXG_MARK(2, 2);
    Dig g[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) load_dig(s_dig, 24 * r + 8 * j + k, g[j]);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) part += dot_iq3(qv[rr][j], aux[rr][j], dd[rr][j], g[j], s_g3, s_sel);
        part += dppf<DPP_XOR1>(part);
        part += dppf<DPP_XOR2>(part);
        part += dppf<DPP_HALF_MIRROR>(part);   // lanes 8q..8q+7 now hold expert rank q's row
        const float y = (ok && isfinite(part)) ? part : 0.0f;
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
                                                                   float *norm_dump, const DevState *st) {
    if (!st->force_head && st->step + 1 < st->n_prompt) return;
    __shared__ uint32_t s_dig[64 * DIG_STRIDE];
    __shared__ double s_red[4];
    DigIn<2048, true> din;
    digits_load(x, norm_w, din);
    const bool ok = block_digits(din, s_dig, s_red, norm_dump);
    for (int i = threadIdx.x; i < 64 * DIG_STRIDE; i += 256) dig[i] = s_dig[i];
    if (threadIdx.x == 0) dig[64 * DIG_STRIDE] = ok ? 1u : 0u;
}

template <int RPW>
__global__ __launch_bounds__(256) void qxk_head(const uint32_t *dig, const uint8_t *ql,
        const uint8_t *qh, const int8_t *sc, const uint16_t *dd, uint32_t vocab, DevState *st, float *logits) {
    if (!st->force_head && st->step + 1 < st->n_prompt) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 3, ib = lane & 7, hh = ib >> 2, k = ib & 3;
    const uint32_t r0 = (blockIdx.x * 4 + wave) * RPW;
    uint4 l0[RPW], l1[RPW], h0[RPW], h1[RPW];
    int s0[RPW], s1[RPW];
    uint32_t d16[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const uint32_t r = min(r0 + rr, vocab - 1);   // tail rows re-read the last row; not stored
        const uint64_t blk = (uint64_t)r * 8 + b;
        const uint4 *lp = reinterpret_cast<const uint4 *>(ql + blk * 128 + 64 * hh + 32 * (k & 1));
        const uint4 *hp = reinterpret_cast<const uint4 *>(qh + blk * 64 + 32 * hh);
        l0[rr] = lp[0]; l1[rr] = lp[1]; h0[rr] = hp[0]; h1[rr] = hp[1];
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
void qxl_qkv(hipStream_t s, const float *x, const float *nw, const QTensor *q, const QTensor *k, const QTensor *v, float *qkv, Timer t) {
    constexpr int RPW = 4;
    qx_launch(qxk_qkv<RPW>, dim3(5120 / (4 * RPW)), dim3(256), 0, s, t, x, nw, q->p0, q->p1, k->p0, k->p1, v->p0, v->p1, qkv);
}
void qxl_oproj(hipStream_t s, const float *ctxv, const QTensor *o, float *x, float *dump, Timer t) {
    constexpr int RPW = 2;
    qx_launch(qxk_oproj<RPW>, dim3(2048 / (4 * RPW)), dim3(256), 0, s, t, ctxv, o->p0, o->p1, x, dump);
}
void qxl_gate_up(hipStream_t s, const float *x, const float *nw, const QTensor *g, const QTensor *u, Tables T,
                 const double *logits, uint32_t experts, DevState *st, float *h, Timer t) {
    constexpr int UPW = 4;
    qx_launch(qxk_gate_up<UPW>, dim3(QXG_TOPK * QXG_FFN / (4 * UPW)), dim3(256), 0, s, t, x, nw,
                       g->p0, g->p1, g->d, u->p0, u->p1, u->d, T, logits, experts, st, h);
}
void qxl_down(hipStream_t s, const float *h, const QTensor *d, Tables T, const DevState *st, float *x, float *dump, Timer t) {
    constexpr int RPW = 2;
    qx_launch(qxk_down<RPW>, dim3(2048 / (4 * RPW)), dim3(256), 0, s, t, h, d->p0, d->p1, d->d, T, st, x, dump);
}
void qxl_head(hipStream_t s, const float *x, const float *nw, const QTensor *w, uint32_t vocab, DevState *st,
              float *logits, float *norm_dump, uint32_t *dig, Timer t) {
    constexpr int RPW = 4;
    hipLaunchKernelGGL(qxk_norm_digits, dim3(1), dim3(256), 0, s, x, nw, dig, norm_dump, st);
    const uint32_t grid = (vocab + 4 * RPW - 1) / (4 * RPW);
    qx_launch(qxk_head<RPW>, dim3(grid), dim3(256), 0, s, t, dig, w->p0, w->p1, (const int8_t *)w->p2, w->d,
                       vocab, st, logits);
}
}
