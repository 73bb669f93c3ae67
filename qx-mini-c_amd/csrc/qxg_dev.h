// Device helpers shared by the decode kernels: exact fp16 decode, DPP lane
// exchanges, the activation digit scheme and the per-format sub-block dots,
// per-head norm/RoPE and the router top-8.  Header-only (internal linkage).
#pragma once
#include "qxg_internal.h"
#include <climits>

#define DEV __device__ __forceinline__

namespace {

// ---------------------------------------------------------------- helpers
// reference qx_fp16_to_f32 (src/qx_format.c:1854-1876): exact, exponent 31 -> +-65504.
// The hardware conversion is exact for every finite half, subnormals included (half
// denormals are kept in the kernels' default float mode); it yields an infinity or a NaN
// exactly when the exponent is 31, and those take +-65504 with the sign of the input bits
// (not of the converted NaN, whose sign the conversion need not keep).
DEV float fp16_exact(uint32_t h) {
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    return __builtin_isfinite(v) ? v : copysignf(65504.0f, __uint_as_float(h << 16));
}
// A half with exponent 31 replaced by +-65504 (0x7bff with its sign), so the plain hardware
// conversion of the result equals fp16_exact of the input for every bit pattern.  The
// persistent decode's row layouts hold their block scales this way (fp16_d<true>).
DEV uint32_t fp16_sat(uint32_t h) {
    return (h & 0x7c00u) == 0x7c00u ? (h & 0x8000u) | 0x7bffu : h;
}
template <bool SAT>
DEV float fp16_d(uint32_t h) {
    if constexpr (SAT) return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    else return fp16_exact(h);
}

// the wave's index in its workgroup, in a scalar register (the divergence analysis
// does not know that threadIdx.x / 64 is the same in every lane of a wave)
DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Loads of weight bytes, read once per token: non-temporal (streaming), so the 1.4 GB a
// token streams does not displace the small tensors read every layer (router rows, KV
// rows, activations) from the caches (measured: 518 -> 539 tok/s).
typedef uint32_t nt4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt2 __attribute__((ext_vector_type(2)));
DEV uint4 ldw4(const void *p) {
    const nt4 v = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint2 ldw2(const void *p) {
    const nt2 v = __builtin_nontemporal_load(reinterpret_cast<const nt2 *>(p));
    return make_uint2(v.x, v.y);
}
DEV uint32_t ldw1(const void *p) { return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p)); }

DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
// a . b with a zero accumulator, the first of a chain: the three-operand form takes the 0
// inline, where the accumulating form the compiler picks needs a register copy of 0 first.
// sdot4s: the chain's first link when z (a constant at each unrolled call site), else sdot4.
DEV int sdot4z(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
DEV int sdot4s(uint32_t a, uint32_t b, int c, bool z) { return z ? sdot4z(a, b) : sdot4(a, b, c); }
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
DEV float wave_total_f(float v) {
    v += dppf<DPP_XOR1>(v); v += dppf<DPP_XOR2>(v); v += dppf<DPP_ROR4>(v); v += dppf<DPP_ROR8>(v);
    return (rdlanef(v, 0) + rdlanef(v, 16)) + (rdlanef(v, 32) + rdlanef(v, 48));
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

// a * b for |a|, |b| < 2^23 (a full-rate 24-bit multiply; the 32-bit integer multiply runs
// at a quarter of the rate).  The dot epilogues' scale factors (< 2^8) and digit-plane sums
// (< 2^18) are in range.
DEV int mul24(int a, int b) { return __mul24(a, b); }

// aH * 65536 + aM * 256 + aL in f32 for digit-plane sums below 2^24 in magnitude.  The
// m and l sums join in integer first: every caller but dot_q6 bounds |aM * 256 + aL|
// below 2^31 (the largest, IQ3_XXS: 32 values x 62 x 128 x 31 x 256 + the l sum, about
// 2.02e9), so the join is exact and its one rounding to f32 is that of the fma
// fmaf(aM, 256, aL).  combine_wide converts each sum (dot_q6's scaled segments reach 2^24).
DEV float combine(int aH, int aM, int aL) {
    return fmaf((float)aH, 65536.0f, (float)(aM * 256 + aL));
}
DEV float combine_wide(int aH, int aM, int aL) {
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
// H1 (q8_k_compat activations): the m and l planes are zero, their dots are skipped.
// SAT: the scale half is stored saturated (fp16_sat), as in the persistent decode's packs.
template <bool H1 = false, bool SAT = false>
DEV float dot_iq4(uint4 qs, uint2 meta, int ib, const Dig &g) {
    const uint32_t sh = meta.x >> 16, sl = meta.y;
    const int ls = ((sl >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
    const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    int aH = 0, aM = 0, aL = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t wlo = kv_lookup(q[k] & 0x0f0f0f0fu);
        const uint32_t whi = kv_lookup((q[k] >> 4) & 0x0f0f0f0fu);
        aH = sdot4s(wlo, g.h[k], aH, k == 0); aH = sdot4(whi, g.h[4 + k], aH);
        if constexpr (!H1) {
            aM = sdot4s(wlo, g.m[k], aM, k == 0); aM = sdot4(whi, g.m[4 + k], aM);
            aL = sdot4s(wlo, g.l[k], aL, k == 0); aL = sdot4(whi, g.l[4 + k], aL);
        }
    }
    const float dl = fp16_d<SAT>(meta.x & 0xffffu) * (float)(ls - 32);
    return (dl * g.s) * combine(aH, aM, aL);
}

// IQ2_XS sub-block (32 values = 4 grid entries of 8): halves scaled d*(2s+1)/8.  Two phases:
// iq2_look issues the sub-block's LDS codebook reads (grid entries and sign selectors),
// iq2_dot does the arithmetic, so a caller can keep the next sub-block's reads in flight
// while it computes this one (one dependent LDS round trip per sub-block, not one per entry).
struct Iq2Look {
    uint4 gg[4];
    uint2 sl[4];
};
DEV void iq2_look(uint2 qs, const uint4 *G2, const uint2 *SEL, Iq2Look &k) {
    const uint32_t qv[4] = {qs.x & 0xffffu, qs.x >> 16, qs.y & 0xffffu, qs.y >> 16};
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        k.gg[l] = G2[qv[l] & 511u];
        k.sl[l] = SEL[qv[l] >> 9];
    }
}
template <bool H1 = false, bool SAT = false>
DEV float iq2_dot(const Iq2Look &k, uint32_t sc, uint32_t d16, const Dig &g) {
    int h0 = 0, m0 = 0, l0 = 0, h1 = 0, m1 = 0, l1 = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t w0 = perm(k.gg[l].z, k.gg[l].x, k.sl[l].x), w1 = perm(k.gg[l].w, k.gg[l].y, k.sl[l].y);
        if (l < 2) {
            h0 = sdot4s(w0, g.h[2 * l], h0, l == 0); h0 = sdot4(w1, g.h[2 * l + 1], h0);
            if constexpr (!H1) {
                m0 = sdot4s(w0, g.m[2 * l], m0, l == 0); m0 = sdot4(w1, g.m[2 * l + 1], m0);
                l0 = sdot4s(w0, g.l[2 * l], l0, l == 0); l0 = sdot4(w1, g.l[2 * l + 1], l0);
            }
        } else {
            h1 = sdot4s(w0, g.h[2 * l], h1, l == 2); h1 = sdot4(w1, g.h[2 * l + 1], h1);
            if constexpr (!H1) {
                m1 = sdot4s(w0, g.m[2 * l], m1, l == 2); m1 = sdot4(w1, g.m[2 * l + 1], m1);
                l1 = sdot4s(w0, g.l[2 * l], l1, l == 2); l1 = sdot4(w1, g.l[2 * l + 1], l1);
            }
        }
    }
    const int k0 = 2 * (int)(sc & 15u) + 1, k1 = 2 * (int)(sc >> 4) + 1;
    const float v = combine(mul24(k0, h0) + mul24(k1, h1), mul24(k0, m0) + mul24(k1, m1), mul24(k0, l0) + mul24(k1, l1));
    return ((fp16_d<SAT>(d16) * 0.125f) * g.s) * v;
}
DEV float dot_iq2(uint2 qs, uint32_t sc, uint32_t d16, const Dig &g, const uint4 *G2, const uint2 *SEL) {
    Iq2Look k;
    iq2_look(qs, G2, SEL, k);
    return iq2_dot(k, sc, d16, g);
}

// IQ3_XXS sub-block: 8 grid indices (4 values each), scale d*(2a+1)/4; iq3_look / iq3_dot
// split as for IQ2_XS.
struct Iq3Look {
    uint2 g[8];
    uint2 sl[4];
};
DEV void iq3_look(uint2 qs, uint32_t aux, const uint2 *G3, const uint2 *SEL, Iq3Look &k) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t word = l < 2 ? qs.x : qs.y;
        k.g[2 * l] = G3[(word >> (16 * (l & 1))) & 255u];
        k.g[2 * l + 1] = G3[(word >> (16 * (l & 1) + 8)) & 255u];
        k.sl[l] = SEL[(aux >> (7 * l)) & 127u];
    }
}
template <bool H1 = false, bool SAT = false>
DEV float iq3_dot(const Iq3Look &k, uint32_t aux, uint32_t d16, const Dig &g) {
    int aH = 0, aM = 0, aL = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t w0 = perm(k.g[2 * l].y, k.g[2 * l].x, k.sl[l].x), w1 = perm(k.g[2 * l + 1].y, k.g[2 * l + 1].x, k.sl[l].y);
        aH = sdot4s(w0, g.h[2 * l], aH, l == 0); aH = sdot4(w1, g.h[2 * l + 1], aH);
        if constexpr (!H1) {
            aM = sdot4s(w0, g.m[2 * l], aM, l == 0); aM = sdot4(w1, g.m[2 * l + 1], aM);
            aL = sdot4s(w0, g.l[2 * l], aL, l == 0); aL = sdot4(w1, g.l[2 * l + 1], aL);
        }
    }
    const int k3 = 2 * (int)(aux >> 28) + 1;
    return ((fp16_d<SAT>(d16) * 0.25f) * g.s) * combine(mul24(k3, aH), mul24(k3, aM), mul24(k3, aL));
}
DEV float dot_iq3(uint2 qs, uint32_t aux, uint32_t d16, const Dig &g, const uint2 *G3, const uint2 *SEL) {
    Iq3Look k;
    iq3_look(qs, aux, G3, SEL, k);
    return iq3_dot(k, aux, d16, g);
}

// IQ2_S sub-block (32 values = 4 grid entries of 8; src/qx_format.c:1961-1984): 10-bit grid
// index qs[l] | (2 bits of the sub-block's qh byte), explicit sign byte per entry,
// halves scaled d*(2s+1)/8 as IQ2_XS.  G2S: 1024 entries {pos lo, pos hi, neg lo, neg hi};
// SEL8: sign byte -> v_perm selectors.
DEV float dot_iq2s(uint32_t qs4, uint32_t sg4, uint32_t qh, uint32_t sc, uint32_t d16, const Dig &g,
                   const uint4 *G2S, const uint2 *SEL8) {
    int h0 = 0, m0 = 0, l0 = 0, h1 = 0, m1 = 0, l1 = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t idx = ((qs4 >> (8 * l)) & 255u) | ((qh << (8 - 2 * l)) & 0x300u);
        const uint4 gg = G2S[idx];
        const uint2 sl = SEL8[(sg4 >> (8 * l)) & 255u];
        const uint32_t w0 = perm(gg.z, gg.x, sl.x), w1 = perm(gg.w, gg.y, sl.y);
        if (l < 2) {
            h0 = sdot4s(w0, g.h[2 * l], h0, l == 0); h0 = sdot4(w1, g.h[2 * l + 1], h0);
            m0 = sdot4s(w0, g.m[2 * l], m0, l == 0); m0 = sdot4(w1, g.m[2 * l + 1], m0);
            l0 = sdot4s(w0, g.l[2 * l], l0, l == 0); l0 = sdot4(w1, g.l[2 * l + 1], l0);
        } else {
            h1 = sdot4s(w0, g.h[2 * l], h1, l == 2); h1 = sdot4(w1, g.h[2 * l + 1], h1);
            m1 = sdot4s(w0, g.m[2 * l], m1, l == 2); m1 = sdot4(w1, g.m[2 * l + 1], m1);
            l1 = sdot4s(w0, g.l[2 * l], l1, l == 2); l1 = sdot4(w1, g.l[2 * l + 1], l1);
        }
    }
    const int k0 = 2 * (int)(sc & 15u) + 1, k1 = 2 * (int)((sc >> 4) & 15u) + 1;
    const float v = combine(mul24(k0, h0) + mul24(k1, h1), mul24(k0, m0) + mul24(k1, m1), mul24(k0, l0) + mul24(k1, l1));
    return ((fp16_exact(d16) * 0.125f) * g.s) * v;
}

// IQ3_S sub-block (src/qx_format.c:1986-2030): 8 grid indices of 9 bits (qs byte | one
// bit of the sub-block's qh byte), 4 values each, explicit sign byte per 8 values,
// scale d*(2s+1) (s = the sub-block's 4-bit scale).  G3S: 512 entries {pos, neg}.
DEV float dot_iq3s(uint2 qs8, uint32_t sg4, uint32_t qh, uint32_t sc, uint32_t d16, const Dig &g,
                   const uint2 *G3S, const uint2 *SEL8) {
    int aH = 0, aM = 0, aL = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t word = l < 2 ? qs8.x : qs8.y;
        const uint32_t b1 = ((word >> (16 * (l & 1))) & 255u) | ((qh << (8 - 2 * l)) & 256u);
        const uint32_t b2 = ((word >> (16 * (l & 1) + 8)) & 255u) | ((qh << (7 - 2 * l)) & 256u);
        const uint2 g1 = G3S[b1], g2 = G3S[b2];
        const uint2 sl = SEL8[(sg4 >> (8 * l)) & 255u];
        const uint32_t w0 = perm(g1.y, g1.x, sl.x), w1 = perm(g2.y, g2.x, sl.y);
        aH = sdot4s(w0, g.h[2 * l], aH, l == 0); aH = sdot4(w1, g.h[2 * l + 1], aH);
        aM = sdot4s(w0, g.m[2 * l], aM, l == 0); aM = sdot4(w1, g.m[2 * l + 1], aM);
        aL = sdot4s(w0, g.l[2 * l], aL, l == 0); aL = sdot4(w1, g.l[2 * l + 1], aL);
    }
    const int k = 2 * (int)(sc & 15u) + 1;
    return (fp16_exact(d16) * g.s) * combine(mul24(k, aH), mul24(k, aM), mul24(k, aL));
}

// Q5_K sub-block ib (src/qx_format.c:2112-2145): values 32ib..32ib+31 have 5-bit codes
// (nibble ib&1 of qs[32*(ib/2) + l]) | (bit ib of qh[l]) << 4 and w = d*sc*code - dmin*m
// (6-bit sc, m of the sub-block, get_scale_min_k4 :2079-2087).  The dot is
// d*sc * sum(code*x) - dmin*m * sum(x), both sums exact over the digits.  qa, qb: the
// 32 qs bytes of the sub-block's 64-value group; ha, hb: the block's 32 qh bytes;
// meta = {d, dmin, scales[12]}.
DEV float dot_q5(uint4 qa, uint4 qb, uint4 ha, uint4 hb, uint4 meta, int ib, const Dig &g) {
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const uint32_t hq[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    const uint32_t nsh = 4 * (ib & 1);
    int aH = 0, aM = 0, aL = 0, sH = 0, sM = 0, sL = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t c = ((q[k] >> nsh) & 0x0f0f0f0fu) | (((hq[k] >> ib) & 0x01010101u) << 4);
        aH = sdot4s(c, g.h[k], aH, k == 0); aM = sdot4s(c, g.m[k], aM, k == 0); aL = sdot4s(c, g.l[k], aL, k == 0);
        sH = sdot4s(0x01010101u, g.h[k], sH, k == 0); sM = sdot4s(0x01010101u, g.m[k], sM, k == 0);
        sL = sdot4s(0x01010101u, g.l[k], sL, k == 0);
    }
    const uint32_t s[3] = {meta.y, meta.z, meta.w};   // scales bytes 0..11
    auto byte = [&](int i) -> uint32_t { return (s[i >> 2] >> (8 * (i & 3))) & 255u; };
    uint32_t sc, mn;
    if (ib < 4) { sc = byte(ib) & 63u; mn = byte(ib + 4) & 63u; }
    else { sc = (byte(ib + 4) & 15u) | ((byte(ib - 4) >> 6) << 4); mn = (byte(ib + 4) >> 4) | ((byte(ib) >> 6) << 4); }
    const float d1 = fp16_exact(meta.x & 0xffffu) * (float)sc, m1 = fp16_exact(meta.x >> 16) * (float)mn;
    return (d1 * g.s) * combine(aH, aM, aL) - (m1 * g.s) * combine(sH, sM, sL);
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

template <bool H1 = false>
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
        if constexpr (!H1) {
            aM[s] = sdot4(u, g.m[j], aM[s]);
            aL[s] = sdot4(u, g.l[j], aL[s]);
        }
    }
    const float v = combine_wide(mul24(sc0, aH[0]) + mul24(sc1, aH[1]), mul24(sc0, aM[0]) + mul24(sc1, aM[1]),
                                 mul24(sc0, aL[0]) + mul24(sc1, aL[1]));
    return (fp16_exact(d16) * g.s) * v;
}

// Q4_K embedding row (8 blocks) -> 2048 floats (reference src/qx_format.c:2079-2110,
// 3759-3793); 256 threads, thread (b, l) produces 8 values of block b.
DEV void embed_q4k_row(const uint8_t *row, float *x) {
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


// Block-wide "no lane has the flag" for 256 threads, ending with the barrier the
// caller needs anyway: each wave's ballot goes to LDS, one barrier, four reads.  One
// use per kernel (a second call could overwrite the words before a slow wave reads them).
DEV bool block_none256(bool flag) {
    __shared__ uint32_t s_any[4];
    const bool any = __ballot(flag) != 0;
    if ((threadIdx.x & 63) == 0) s_any[threadIdx.x >> 6] = any ? 1u : 0u;
    __syncthreads();
    return (s_any[0] | s_any[1] | s_any[2] | s_any[3]) == 0u;
}

// ---- block-cooperative activation digits.  The digit planes of all N/32 groups of
// a vector are computed once per block into LDS (DIG_STRIDE dwords per group: h[8],
// m[8], l[8], scale bits), 8 consecutive values per thread; the 4 threads of a group
// form a quad, so the group max is two in-quad DPP exchanges.  With NORM, the vector
// is first RMS-normalised with weights w (reference src/qx_format.c:3358-3371).
constexpr int DIG_STRIDE = 28;   // 16-byte aligned rows for ds_read_b128

// X = rint(y * 2^k) with k = 22 - e (e the exponent of the group max, 2^(e-1) <= mx < 2^e),
// so |X| <= 2^22: one fma adds 1.5 * 2^23, whose binade has unit spacing, and the
// integer is the difference of the bit patterns.  k is capped at 126 so 2^k and the
// scale 2^-k stay normal floats (groups below 2^-104 keep fewer than 22 bits).  A
// non-finite group (mx passed as 0) gives p2 = 0; its values are discarded by the
// caller's finiteness flag.  Digits: L = X mod 256 (signed), M the next byte of
// (X - L) / 256, H = the rest, each in [-128, 127].  They come out of one subtraction:
// X + 0x808080 (in [0, 2^24) for |X| <= 2^22) has bytes L + 128, M + 128, H + 128 (the
// bias absorbs every borrow), so a byte transpose of four values and an XOR with 0x80 per
// byte give the three planes.
DEV void digits8(const float *y, float mx, uint32_t &ph0, uint32_t &ph1, uint32_t &pm0, uint32_t &pm1, uint32_t &pl0,
                 uint32_t &pl1, float &scale) {
    int e = 0;
    if (mx > 0.0f) (void)frexpf(mx, &e);
    const int k = min(22 - e, 126);
    const float p2 = mx > 0.0f ? __uint_as_float((uint32_t)(k + 127) << 23) : 0.0f;
    scale = mx > 0.0f ? __uint_as_float((uint32_t)(127 - k) << 23) : 0.0f;
    uint32_t xb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xb[i] = __float_as_uint(fmaf(y[i], p2, 12582912.0f)) - (0x4B400000u - 0x808080u);
    // values v0..v3 -> [v0 b0, v1 b0, v0 b1, v1 b1] and [v0 b2, v1 b2, 0, 0] per pair, then merges
    uint32_t pl[2], pm[2], ph[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t *v = xb + 4 * q;
        const uint32_t t0 = perm(v[1], v[0], 0x05010400u), t1 = perm(v[3], v[2], 0x05010400u);
        const uint32_t u0 = perm(v[1], v[0], 0x0c0c0602u), u1 = perm(v[3], v[2], 0x0c0c0602u);
        pl[q] = perm(t1, t0, 0x05040100u) ^ 0x80808080u;
        pm[q] = perm(t1, t0, 0x07060302u) ^ 0x80808080u;
        ph[q] = perm(u1, u0, 0x05040100u) ^ 0x80808080u;
    }
    pl0 = pl[0]; pl1 = pl[1]; pm0 = pm[0]; pm1 = pm[1]; ph0 = ph[0]; ph1 = ph[1];
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
    // every thread of the 256 loads its chunks unconditionally: straight-line loads let
    // the compiler wait for each one separately (a load under a branch makes it wait for
    // every load issued before the branch joins)
    static_assert(D::NCH == 256 * D::PER, "the 256 threads cover the vector exactly");
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < D::PER; ++it) {
        const int c = tid + 256 * it;
        const float4 a = reinterpret_cast<const float4 *>(x)[2 * c], b = reinterpret_cast<const float4 *>(x)[2 * c + 1];
        in.v[it][0] = a.x; in.v[it][1] = a.y; in.v[it][2] = a.z; in.v[it][3] = a.w;
        in.v[it][4] = b.x; in.v[it][5] = b.y; in.v[it][6] = b.z; in.v[it][7] = b.w;
    }
    if constexpr (NORM) {
        static_assert(D::PER == 1, "normalised vectors are 2048 long");
        const float4 a = reinterpret_cast<const float4 *>(w)[2 * tid], b = reinterpret_cast<const float4 *>(w)[2 * tid + 1];
        in.w[0] = a.x; in.w[1] = a.y; in.w[2] = a.z; in.w[3] = a.w;
        in.w[4] = b.x; in.w[5] = b.y; in.w[6] = b.z; in.w[7] = b.w;
    }
}

// RMSNorm of a 2048-vector held 8 values per thread (src/qx_format.c:3358-3371)
template <int N>
DEV void rms_normalise(DigIn<N, true> &in, double *s_red, float *norm_out) {
    const int tid = threadIdx.x;
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

// returns true when every value is finite (block-uniform); ends with a block barrier
template <int N, bool NORM>
DEV bool block_digits(DigIn<N, NORM> &in, uint32_t *s_dig, double *s_red, float *norm_out = nullptr) {
    using D = DigIn<N, NORM>;
    const int tid = threadIdx.x;
    if constexpr (NORM) rms_normalise(in, s_red, norm_out);
    bool fin = true;
#pragma unroll
    for (int it = 0; it < D::PER; ++it) {
        const int c = tid + 256 * it;
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) { fin = fin && isfinite(in.v[it][i]); mx = fmaxf(mx, fabsf(in.v[it][i])); }
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
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
    return block_none256(!fin);
}

// q8_k_compat activations (src/qx_format.c:3891-3927).  A 256-value block is the 8
// values of each of 32 consecutive lanes (half a wave): the value of largest magnitude,
// first on ties, maps to -127: inv = -127/max, d = 1/inv, code = round-half-even(inv * v)
// clamped to [-128, 127].  Every lane of the wave must call this (it exchanges lanes).
// Returns d; the lane's 8 codes are packed in h0 (values 0-3) and h1 (4-7).
DEV float q8_chunk(const float (&v)[8], uint32_t &h0, uint32_t &h1) {
    const int half = (threadIdx.x & 63) >> 5;
    float am = 0.0f, vm = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (fabsf(v[i]) > am) { am = fabsf(v[i]); vm = v[i]; }
    // the half-wave's largest magnitude: each 16-lane row's by DPP, then the two rows' read
    // out (no LDS round trip); the first lane holding it, per half, from one ballot
    float bm = fmaxf(am, dppf<DPP_XOR1>(am));
    bm = fmaxf(bm, dppf<DPP_XOR2>(bm));
    bm = fmaxf(bm, dppf<DPP_ROR4>(bm));
    bm = fmaxf(bm, dppf<DPP_ROR8>(bm));
    const float b0 = fmaxf(rdlanef(bm, 0), rdlanef(bm, 16)), b1 = fmaxf(rdlanef(bm, 32), rdlanef(bm, 48));
    bm = half ? b1 : b0;
    const uint64_t hits = __ballot(am == bm);
    const uint32_t lo = (uint32_t)hits, hi = (uint32_t)(hits >> 32);
    const float v0 = rdlanef(vm, lo ? __ffs(lo) - 1 : 0), v1 = rdlanef(vm, hi ? 31 + __ffs(hi) : 32);
    const float vmax = half ? v1 : v0;
    const float inv = vmax == 0.0f ? 0.0f : -127.0f / vmax;
    uint32_t H[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int q = inv == 0.0f ? 0 : (int)rintf(inv * v[i]);
        q = q > 127 ? 127 : q < -128 ? -128 : q;
        H[i >> 2] |= (uint32_t)(q & 255) << (8 * (i & 3));
    }
    h0 = H[0];
    h1 = H[1];
    return inv == 0.0f ? 0.0f : 1.0f / inv;
}

// Q8_K activations in the digit-plane layout: codes in the h plane, m = l = 0, and every
// 32-group of a block carries the scale d/65536, so the digit dots compute d * sum(code
// * w).  Returns true when every value is finite (block-uniform); ends with a barrier.
template <int N, bool NORM>
DEV bool block_q8(DigIn<N, NORM> &in, uint32_t *s_dig, double *s_red, float *norm_out = nullptr) {
    using D = DigIn<N, NORM>;
    static_assert(D::NCH % 32 == 0, "each 256-value block is the 32 chunks of one half-wave");
    const int tid = threadIdx.x;
    if constexpr (NORM) rms_normalise(in, s_red, norm_out);
    bool fin = true;
#pragma unroll
    for (int it = 0; it < D::PER; ++it) {
        const int c = tid + 256 * it;
#pragma unroll
        for (int i = 0; i < 8; ++i) fin = fin && isfinite(in.v[it][i]);
        uint32_t h0, h1;
        const float dq = q8_chunk(in.v[it], h0, h1);
        uint32_t *d = s_dig + (c >> 2) * DIG_STRIDE;
        const int q = c & 3;
        *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
        *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(0u, 0u);
        *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(0u, 0u);
        if (q == 0) d[24] = __float_as_uint(dq * (1.0f / 65536.0f));
    }
    return block_none256(!fin);
}

// the activation mode's preparation: Q8_K codes, or the three-plane digits of f32
template <bool Q8, int N, bool NORM>
DEV bool block_act(DigIn<N, NORM> &in, uint32_t *s_dig, double *s_red, float *norm_out = nullptr) {
    if constexpr (Q8) return block_q8(in, s_dig, s_red, norm_out);
    else return block_digits(in, s_dig, s_red, norm_out);
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
// a prompt step whose logits nobody reads (the head kernels skip it).  The fields are
// read together, not behind a short-circuit, so they come in one scalar load.
DEV bool prompt_step(const DevState *st) {
    const uint32_t fh = st->force_head, step = st->step, np = st->n_prompt;
    return (fh == 0u) & (step + 1u < np);
}

// The sum of v over the wave's four 16-lane rows, in every lane: v_permlane32_swap
// exchanges the upper half of one register with the lower half of another (each lane then
// adds the value 32 lanes away), v_permlane16_swap the odd rows with the even ones.  Every
// lane forms the same two sums in the same order, so the result is uniform.
DEV float rows4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The same sum in the order of xor-16 then xor-32 shuffles, (row 0 + row 1) + (row 2 + row 3)
// in every lane, bit for bit what two __shfl_xor steps give, without their LDS round trips.
DEV float rows4_sum_pairs(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// R per-lane partial sums (one per row, R in {1,2,4,8}) reduced over the wave:
// up to two split rounds inside each quad (a lane keeps half of the rows and adds
// its partner's half), then row16 sums, then the four 16-lane rows (rows4_sum) and
// one readlane per row.  out[r] is the total of row r, wave-uniform.
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
        v[i] = rows4_sum(v[i]);
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
        out[r] = rdlanef(t, l0);
    }
}


DEV float block_max256(float v, float *red) {
    v = fmaxf(v, dppf<DPP_XOR1>(v)); v = fmaxf(v, dppf<DPP_XOR2>(v));
    v = fmaxf(v, dppf<DPP_ROR4>(v)); v = fmaxf(v, dppf<DPP_ROR8>(v));
    v = fmaxf(fmaxf(rdlanef(v, 0), rdlanef(v, 16)), fmaxf(rdlanef(v, 32), rdlanef(v, 48)));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// block maxima of two values at once, one barrier; red[4] must not be in use (no
// earlier phase of the block reads it after its last barrier)
DEV void block_max2_256(float &a, float &b, float2 *red) {
    a = fmaxf(a, dppf<DPP_XOR1>(a)); b = fmaxf(b, dppf<DPP_XOR1>(b));
    a = fmaxf(a, dppf<DPP_XOR2>(a)); b = fmaxf(b, dppf<DPP_XOR2>(b));
    a = fmaxf(a, dppf<DPP_ROR4>(a)); b = fmaxf(b, dppf<DPP_ROR4>(b));
    a = fmaxf(a, dppf<DPP_ROR8>(a)); b = fmaxf(b, dppf<DPP_ROR8>(b));
    a = fmaxf(fmaxf(rdlanef(a, 0), rdlanef(a, 16)), fmaxf(rdlanef(a, 32), rdlanef(a, 48)));
    b = fmaxf(fmaxf(rdlanef(b, 0), rdlanef(b, 16)), fmaxf(rdlanef(b, 32), rdlanef(b, 48)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = make_float2(a, b);
    __syncthreads();
    const float2 r0 = red[0], r1 = red[1], r2 = red[2], r3 = red[3];
    a = fmaxf(fmaxf(r0.x, r1.x), fmaxf(r2.x, r3.x));
    b = fmaxf(fmaxf(r0.y, r1.y), fmaxf(r2.y, r3.y));
}

// INT8 KV quantization of one row (reference qx_quantize_int8_vector, src/qx_format.c:4449-4463):
// scale = max |x| / 127 over the finite values (1 if that is 0), code = lrintf(x / scale) with
// the f32 division correctly rounded (the build flag) and round-half-even, clamped to +-127,
// non-finite -> 0.  Every kernel that appends a KV row quantizes with these two functions (the
// maximum itself is exact in any order); qxg_int8_quantize runs them on a given row.
DEV float int8_mag(float x) { return isfinite(x) ? fabsf(x) : 0.0f; }
DEV float int8_scale(float max_abs) { return max_abs > 0.0f ? max_abs / 127.0f : 1.0f; }
DEV int8_t int8_code(float x, float scale) {
    const int q = isfinite(x) ? (int)rintf(x / scale) : 0;
    return (int8_t)(q < -127 ? -127 : q > 127 ? 127 : q);
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

// ---- GQA attention of one q head over cached INT8 positions 0..n-1 by a block of 256
// threads (qx_rope_gqa_attention_partial, src/qx_format.c:5051-5196).
// q (128 f32 in LDS) is written as int8 digit planes per group of 32 dimensions
// (22 significant bits, as the projections' activations), so the score of a position is
// exact int32 v_dot4 sums of those digits with the position's INT8 K codes:
//     score = ks * sum_g s_g * (2^16 H_g.k + 2^8 M_g.k + L_g.k) / sqrt(hd),
// non-finite (or a non-finite q) -> 0.  Four lanes per position; krow(t, g, k[2], ks)
// fetches the 32 K bytes of group g of position t and the scale.  s_sc[t] <- score;
// returns the block maximum (wave maxima in redd[0..3]; attn_weights uses redd[4..7]).
template <typename KF>
DEV double attn_scores(const float *s_q, uint32_t *s_qd, uint32_t n, double sqrt_hd, double *s_sc, double *redd,
                       KF krow) {
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    bool fin = true;
    if (tid < 16) {   // 4 groups x 4 threads of 8 values (quads: the group max is two DPP steps)
        float y[8];
        const float4 a = *reinterpret_cast<const float4 *>(s_q + 8 * tid), b = *reinterpret_cast<const float4 *>(s_q + 8 * tid + 4);
        y[0] = a.x; y[1] = a.y; y[2] = a.z; y[3] = a.w; y[4] = b.x; y[5] = b.y; y[6] = b.z; y[7] = b.w;
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) { fin = fin && isfinite(y[i]); mx = fmaxf(mx, fabsf(y[i])); }
        mx = fmaxf(mx, dppf<DPP_XOR1>(mx));
        mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
        uint32_t h0, h1, m0, m1, l0, l1;
        float sc;
        digits8(y, fin && isfinite(mx) ? mx : 0.0f, h0, h1, m0, m1, l0, l1, sc);
        uint32_t *d = s_qd + (tid >> 2) * DIG_STRIDE;
        const int q = tid & 3;
        *reinterpret_cast<uint2 *>(d + 2 * q) = make_uint2(h0, h1);
        *reinterpret_cast<uint2 *>(d + 8 + 2 * q) = make_uint2(m0, m1);
        *reinterpret_cast<uint2 *>(d + 16 + 2 * q) = make_uint2(l0, l1);
        if (q == 0) d[24] = __float_as_uint(sc);
    }
    const bool qok = block_none256(!fin);
    // a quad per position: lane q4 of the quad takes the 32-dim group q4, the four group
    // sums are added as (g0 + g1) + (g2 + g3) in double
    const int q4 = tid & 3;
    Dig d;
    load_dig(s_qd, q4, d);
    double mx = -1.0e300;
    for (uint32_t t = tid >> 2; t < n; t += 64) {
        uint4 k[2];
        float ksc;
        krow(t, q4, k, ksc);
        const uint32_t kw[8] = {k[0].x, k[0].y, k[0].z, k[0].w, k[1].x, k[1].y, k[1].z, k[1].w};
        int aH = 0, aM = 0, aL = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            aH = sdot4s(kw[i], d.h[i], aH, i == 0);
            aM = sdot4s(kw[i], d.m[i], aM, i == 0);
            aL = sdot4s(kw[i], d.l[i], aL, i == 0);
        }
        double acc = (double)(combine(aH, aM, aL) * d.s);
        acc += dppd<DPP_XOR1>(acc);   // the quad shares t, so its lanes are active together
        acc += dppd<DPP_XOR2>(acc);
        double sc = qok ? acc * (double)ksc / sqrt_hd : 0.0;
        if (!isfinite(sc)) sc = 0.0;
        if (q4 == 0) s_sc[t] = sc;
        mx = fmax(mx, sc);
    }
    mx = wave_max_d(mx);
    if (lane == 0) redd[wave] = mx;
    __syncthreads();
    return fmax(fmax(redd[0], redd[1]), fmax(redd[2], redd[3]));   // redd[0..3] not written again
}
// Softmax in double: e_t = exp(s_t - mx), den = sum e_t (1 if not finite and positive);
// s_sc[t] <- (e_t / den) * vs_t, the position's weight with its V scale folded in.
// Unnormalised (norm false, one split of several): s_sc[t] <- e_t * vs_t and the raw
// den is returned.  vsc(t) returns position t's V scale.  Ends with a barrier.
template <typename VS>
DEV double attn_weights(uint32_t n, double mx, double *s_sc, double *redd, VS vsc, bool norm = true,
                        double *wsum = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    double den = 0.0;
    for (uint32_t t = tid; t < n; t += 256) {
        const double e = exp(s_sc[t] - mx);
        s_sc[t] = e;
        den += e;
    }
    den = wave_total_d(den);
    if (lane == 0) redd[4 + wave] = den;   // redd[0..3] may still be read by the score maximum
    __syncthreads();
    den = (redd[4] + redd[5]) + (redd[6] + redd[7]);
    double ws = 0.0;   // the head's sum of normalised weights (a diagnostic, when wsum is given)
    if (norm) {
        if (!isfinite(den) || den <= 0.0) den = 1.0;
        for (uint32_t t = tid; t < n; t += 256) {
            const double w = s_sc[t] / den;
            ws += w;
            s_sc[t] = w * (double)vsc(t);
        }
    } else {
        for (uint32_t t = tid; t < n; t += 256) s_sc[t] = s_sc[t] * (double)vsc(t);
    }
    __syncthreads();
    if (wsum && norm) {   // block-uniform; redd[0..3] are free after the barrier above
        ws = wave_total_d(ws);
        if (lane == 0) redd[wave] = ws;
        __syncthreads();
        if (tid == 0) *wsum = (redd[0] + redd[1]) + (redd[2] + redd[3]);
        __syncthreads();
    }
    return den;
}
// Context: out[d] = sum_t p_t * v8_t[d] in f32 with p_t = (float)((e_t / den) * vs_t).
// Thread (g = tid/16, dims 8*(tid%16)..+8) sums positions g, g+16, ...; the 16 partial
// sums of a dimension are then added in g order.  vrow(t, dg) returns the 8 V bytes.
template <typename VF>
DEV void attn_context(uint32_t n, const double *s_sc, float (*s_part)[132], VF vrow, float *out) {
    const int tid = threadIdx.x, g = tid >> 4, dg = tid & 15;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll 4
    for (uint32_t t = g; t < n; t += 16) {
        const float p = (float)s_sc[t];
        const uint2 v = vrow(t, dg);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int8_t vb = (int8_t)((((j < 4) ? v.x : v.y) >> (8 * (j & 3))) & 255u);
            acc[j] = fmaf(p, (float)vb, acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s_part[g][8 * dg + j] = acc[j];
    __syncthreads();
    if (tid < 128) {
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) o += s_part[i][tid];
        out[tid] = o;
    }
}

// order-preserving unsigned image of a double: a > b  <=>  key(a) > key(b); NaN -> 0,
// below every number
DEV uint64_t dkey(double v) {
    if (v != v) return 0ull;
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
template <int CTRL>
DEV uint64_t dppu64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}
DEV uint64_t rdlaneu64(uint64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}
DEV uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
// wave-uniform maximum of a 64-bit key
DEV uint64_t wave_max_u64(uint64_t v) {
    v = umax64(v, dppu64<DPP_XOR1>(v)); v = umax64(v, dppu64<DPP_XOR2>(v));
    v = umax64(v, dppu64<DPP_ROR4>(v)); v = umax64(v, dppu64<DPP_ROR8>(v));
    return umax64(umax64(rdlaneu64(v, 0), rdlaneu64(v, 16)), umax64(rdlaneu64(v, 32), rdlaneu64(v, 48)));
}

// order-preserving unsigned image of (float)v (f32 rounding is monotone); NaN -> 0
DEV uint32_t fkey(double v) {
    const float f = (float)v;
    if (f != f) return 0u;
    const uint32_t b = __float_as_uint(f);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}
DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dppi<DPP_XOR1>((int)v)); v = max(v, (uint32_t)dppi<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dppi<DPP_ROR4>((int)v)); v = max(v, (uint32_t)dppi<DPP_ROR8>((int)v));
    return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
               max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

// 8 rounds of "largest key, lowest expert index among equal keys, then retire it";
// returns true when some round had several experts at the maximum key.
template <typename K, typename MaxF>
DEV bool top8_rounds(K k0, K k1, MaxF wmax, uint32_t (&ids)[QXG_TOPK]) {
    const int lane = threadIdx.x & 63;
    bool tie = false;
#pragma unroll
    for (int r = 0; r < QXG_TOPK; ++r) {
        const K m = wmax(k0 > k1 ? k0 : k1);
        const uint64_t b0 = __ballot(m != 0 && k0 == m), b1 = __ballot(m != 0 && k1 == m);
        tie = tie || (__popcll(b0) + __popcll(b1) > 1);
        // nothing left (non-finite logits): expert 0, as the reference's scan leaves it
        const uint32_t id = b0 ? (uint32_t)__builtin_ctzll(b0) : b1 ? 64u + (uint32_t)__builtin_ctzll(b1) : 0u;
        ids[r] = id;
        if (lane == (int)(id & 63u)) {
            if (id < 64u) k0 = 0; else k1 = 0;
        }
    }
    return tie;
}

// The top 8 of the 128 keys by merging sorted lists across lanes, in a short dependency chain
// (about 30 dependent steps against about 120 for eight rounds of wave maxima; measured 0.71
// against 1.22 us per call).  Keys are packed as the f32 key's top 25 bits over the expert
// index (127 - e, so a lower index wins between equal prefixes), unique, so the list merges
// need no tie handling.  Each lane starts with its two keys as a sorted list; xor-1 and xor-2
// lane exchanges merge the lists to 4 and 8 entries, then four merges keep the top 8 of two
// 8-lists (row rotations by 4 and 8, row broadcasts 15 and 31); lane 63 ends with the wave's
// top 8 in order.  Returns true when the packed order may differ from the order by
// (f32 key, index): two keys of the top 8, or the 8th and a key outside, share a 25-bit
// prefix; the caller then redoes the selection exactly.
#define QXG_CE(x, y) { const uint32_t hi_ = max(x, y), lo_ = min(x, y); x = hi_; y = lo_; }
template <int CTRL, int ROWS>
DEV uint32_t lane_pull(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, false); }
template <int CTRL, int ROWS>
DEV void merge_top8(uint32_t (&v)[8]) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = lane_pull<CTRL, ROWS>(v[i]);   // rows outside ROWS pull 0
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = max(v[i], b[7 - i]);   // the top 8 of both lists, bitonic
    QXG_CE(v[0], v[4]) QXG_CE(v[1], v[5]) QXG_CE(v[2], v[6]) QXG_CE(v[3], v[7])
    QXG_CE(v[0], v[2]) QXG_CE(v[1], v[3]) QXG_CE(v[4], v[6]) QXG_CE(v[5], v[7])
    QXG_CE(v[0], v[1]) QXG_CE(v[2], v[3]) QXG_CE(v[4], v[5]) QXG_CE(v[6], v[7])
}
DEV bool top8_lists(double l0, double l1, int E, uint32_t (&ids)[QXG_TOPK]) {
    static_assert(QXG_TOPK == 8, "eight picks");
    const int lane = threadIdx.x & 63;
    const uint32_t f0 = lane < E ? fkey(l0) : 0u, f1 = lane + 64 < E ? fkey(l1) : 0u;
    const uint32_t k0 = f0 ? (f0 & ~127u) | (127u - (uint32_t)lane) : 0u;
    const uint32_t k1 = f1 ? (f1 & ~127u) | (63u - (uint32_t)lane) : 0u;
    uint32_t v[8] = {max(k0, k1), min(k0, k1), 0u, 0u, 0u, 0u, 0u, 0u};
    {   // 2 + 2 -> 4 (lane xor 1): a0 a1 b1 b0 is bitonic
        const uint32_t b0 = lane_pull<0xb1, 0xf>(v[0]), b1 = lane_pull<0xb1, 0xf>(v[1]);
        v[2] = b1; v[3] = b0;
        QXG_CE(v[0], v[2]) QXG_CE(v[1], v[3]) QXG_CE(v[0], v[1]) QXG_CE(v[2], v[3])
    }
    {   // 4 + 4 -> 8 (lane xor 2)
        uint32_t b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) b[i] = lane_pull<0x4e, 0xf>(v[i]);
        v[4] = b[3]; v[5] = b[2]; v[6] = b[1]; v[7] = b[0];
        QXG_CE(v[0], v[4]) QXG_CE(v[1], v[5]) QXG_CE(v[2], v[6]) QXG_CE(v[3], v[7])
        QXG_CE(v[0], v[2]) QXG_CE(v[1], v[3]) QXG_CE(v[4], v[6]) QXG_CE(v[5], v[7])
        QXG_CE(v[0], v[1]) QXG_CE(v[2], v[3]) QXG_CE(v[4], v[5]) QXG_CE(v[6], v[7])
    }
    merge_top8<0x124, 0xf>(v);   // row_ror:4
    merge_top8<0x128, 0xf>(v);   // row_ror:8: every lane holds its row's top 8
    merge_top8<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    merge_top8<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3: lane 63 holds the wave's
    uint32_t m[8];
    bool tie = false;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        m[q] = (uint32_t)__builtin_amdgcn_readlane((int)v[q], 63);
        ids[q] = m[q] ? 127u - (m[q] & 127u) : 0u;   // no key left (non-finite logits): expert 0
        if (q > 0) tie = tie || (m[q] != 0u && (m[q] & ~127u) == (m[q - 1] & ~127u));
    }
    const uint32_t p7 = m[7] & ~127u;
    return tie || __ballot(p7 != 0u && ((k0 < m[7] && (k0 & ~127u) == p7) || (k1 < m[7] && (k1 & ~127u) == p7))) != 0;
}
#undef QXG_CE

// Router top-8 and renormalised weights (src/qx_format.c:5265-5285), by every wave on
// its own (no block barrier).  Lane l holds the logits of experts l and l+64 (double).
// The reference picks by softmax probability with repeated strict-> scans (larger
// first, lower index on ties); the probability is a non-decreasing function of the
// logit, so picking by logit gives the same experts except where two probabilities
// round to the same double (a zero margin).  The picks use 32-bit keys of the logits
// rounded to f32: a unique maximal f32 key is also the maximal double.  The list merge
// above picks first; where its packed keys may misorder, eight rounds of wave maxima over
// the full f32 keys pick, and only when a round sees several experts at the maximal f32
// key are the picks redone with the exact 64-bit keys of the doubles.  The weights p_r / sum_q p_q equal
// e_r / sum_q e_q with e = exp(l - l_max), since the softmax denominator cancels.
// ids[r] and w[r] are wave-uniform.
DEV void wave_top8_ids(double l0, double l1, int E, uint32_t (&ids)[QXG_TOPK]) {
    const int lane = threadIdx.x & 63;
    if (!top8_lists(l0, l1, E, ids)) return;
    const bool tie = top8_rounds<uint32_t>(lane < E ? fkey(l0) : 0u, lane + 64 < E ? fkey(l1) : 0u,
                                           [](uint32_t v) { return wave_max_u32(v); }, ids);
    if (tie)
        (void)top8_rounds<uint64_t>(lane < E ? dkey(l0) : 0ull, lane + 64 < E ? dkey(l1) : 0ull,
                                    [](uint64_t v) { return wave_max_u64(v); }, ids);
}
// F32EXP: e = exp(x) as (double)expf(hi) * (1 + lo), x = hi + lo with hi = (float)x (relative
// error ~1 f32 ulp, 6e-8, against the double exp; the persistent decode, where a double exp's
// polynomial constants would be held in registers across its layer loop)
template <bool F32EXP = false>
DEV void wave_top8_weights(double l0, double l1, const uint32_t (&ids)[QXG_TOPK], double (&w)[QXG_TOPK]) {
    const int lane = threadIdx.x & 63;
    double lq = 0.0;   // lane q < 8: logit of pick q
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) {
        const double v = ids[q] < 64u ? rdlaned(l0, (int)ids[q]) : rdlaned(l1, (int)(ids[q] - 64u));
        if (lane == q) lq = v;
    }
    const double lmax = rdlaned(lq, 0);
    double eq = 0.0;
    if (lane < QXG_TOPK) {
        const double x = lq - lmax;
        if constexpr (F32EXP) {
            const float hi = (float)x;
            eq = (double)expf(hi) * (1.0 + (x - (double)hi));
        } else {
            eq = exp(x);
        }
    }
    double sel = 0.0;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) sel += rdlaned(eq, q);   // rank order, as the reference
    const double wq = eq / sel;
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q) w[q] = rdlaned(wq, q);
}
DEV void wave_top8(double l0, double l1, int E, uint32_t (&ids)[QXG_TOPK], double (&w)[QXG_TOPK]) {
    wave_top8_ids(l0, l1, E, ids);
    wave_top8_weights(l0, l1, ids, w);
}
}  // namespace
