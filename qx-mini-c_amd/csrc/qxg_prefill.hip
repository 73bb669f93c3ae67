// Batched prefill (CDNA4, gfx950): the T tokens of a prompt chunk go through each
// layer together.  The reference runs a prompt one token at a time through its
// decode step (src/qx_format.c:6250-6547 of the reference); here every projection
// and every expert matrix is one GEMM over the tokens (or over the tokens routed to
// that expert) on the matrix cores.
//
// Precision scheme of the GEMMs (fp16 MFMA 32x32x16, f32 accumulation).  Every
// weight of the formats used is, exactly,
//     IQ2_XS   w = (d/8) * [(2s+1) * grid * sign]        |code| <= 31*43 = 1333
//     IQ3_XXS  w = (d/4) * [(2a+1) * grid * sign]        |code| <= 31*62 = 1922
//     IQ4_XS   w = (d*(ls-32)) * kvalue                  |code| <= 127
// (the f32 products the reference forms, src/qx_format.c:1914-2053, are exact), and
// each bracketed integer code is exact in fp16.  Each activation row is scaled by a
// power of two s (max |x*s| in [2^13, 2^14)) and split as x*s = hi + lo (+ e), hi and
// lo fp16, |e| <= 2^-22 |x*s|.  A code times an fp16 value is exact in f32; the matrix
// cores sum the products in f32 over one block (IQ2_XS, IQ3_XXS: 256 values) or one
// group (IQ4_XS: 32 values), that partial sum is multiplied by its f32 scale once, and
// the row result is divided by s.  The integer codes come from fp16 codebooks in LDS.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane l holds, for A, row l%32 and
// k = 8*(l/32) + j (j < 8); for B, column l%32 and the same k; result register r of
// lane l is (row 8*(r/4) + 4*(l/32) + r%4, column l%32).  Rows are tokens (or expert
// slots), columns are weight rows, so each lane's results share one weight row and
// its scale.  Activations are packed once per GEMM in exactly this fragment order:
//     apk[((mtile * KS + kstep) * 2 + piece) * 64 + lane] = 8 fp16 values (uint4).
#include "qxg_dev.h"

namespace {
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

enum { FMT_IQ4 = 0, FMT_IQ2 = 1, FMT_IQ3 = 2, FMT_Q5 = 3, FMT_IQ2S = 4, FMT_IQ3S = 5 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

DEV f16x mfma(uint4 a, uint4 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
}

DEV uint32_t hmul2(uint32_t v, h2v m) { return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, v) * m); }
DEV uint4 hmul8(uint4 v, uint32_t mul) {
    const _Float16 f = (_Float16)(float)mul;   // 1..31: exact
    const h2v m = {f, f};
    return make_uint4(hmul2(v.x, m), hmul2(v.y, m), hmul2(v.z, m), hmul2(v.w, m));
}
DEV uint32_t comp(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// ---------------------------------------------------------------- weight blocks per lane
// The lane's share of one 256-value block of its weight row: lane half h = l/32 takes
// k = 16*s + 8*h + j of every k-step s (16 per block).
template <int F> struct Blk;
template <> struct Blk<FMT_IQ2> { uint4 q[4]; uint2 sc; uint32_t d; };    // qs (32 x u16), scales, d
template <> struct Blk<FMT_IQ3> { uint4 q[4]; uint4 a[2]; uint32_t d; };  // qs (64 x u8), aux (8 x u32), d
template <> struct Blk<FMT_IQ4> { uint2 q[8]; uint2 m; };                 // qs bytes 16ib+8h..+8, meta
template <> struct Blk<FMT_Q5> { uint2 q[8]; uint2 qh[2]; uint4 m; };     // qs 32p+16t+8h..+8, qh 16t+8h..+8, meta
template <> struct Blk<FMT_IQ2S> { uint4 g[2], sg[2]; uint2 qh, sc; uint32_t d; };   // grid, sign, qh, scale bytes
template <> struct Blk<FMT_IQ3S> { uint4 q[4], sg[2], hs; uint32_t d; };  // grid, sign bytes, {qh[8], scales[4]}

DEV void blk_load(Blk<FMT_IQ2> &b, const PfMat &w, uint64_t bi, int) {
    const uint4 *p = reinterpret_cast<const uint4 *>(w.qs + bi * 64);
    b.q[0] = p[0]; b.q[1] = p[1]; b.q[2] = p[2]; b.q[3] = p[3];
    b.sc = *reinterpret_cast<const uint2 *>(w.p1 + bi * 8);
    b.d = w.d[bi];
}
DEV void blk_load(Blk<FMT_IQ3> &b, const PfMat &w, uint64_t bi, int) {
    const uint4 *p = reinterpret_cast<const uint4 *>(w.qs + bi * 64);
    b.q[0] = p[0]; b.q[1] = p[1]; b.q[2] = p[2]; b.q[3] = p[3];
    const uint4 *a = reinterpret_cast<const uint4 *>(w.p1 + bi * 32);
    b.a[0] = a[0]; b.a[1] = a[1];
    b.d = w.d[bi];
}
DEV void blk_load(Blk<FMT_IQ4> &b, const PfMat &w, uint64_t bi, int h) {
    const uint8_t *q = w.qs + bi * 128 + 8 * h;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) b.q[ib] = *reinterpret_cast<const uint2 *>(q + 16 * ib);
    b.m = *reinterpret_cast<const uint2 *>(w.p1 + bi * 8);
}

DEV void blk_load(Blk<FMT_Q5> &b, const PfMat &w, uint64_t bi, int h) {
    const uint8_t *q = w.qs + bi * 128 + 8 * h;
#pragma unroll
    for (int i = 0; i < 8; ++i) b.q[i] = *reinterpret_cast<const uint2 *>(q + 32 * (i >> 1) + 16 * (i & 1));
    b.qh[0] = *reinterpret_cast<const uint2 *>(w.p2 + bi * 32 + 8 * h);
    b.qh[1] = *reinterpret_cast<const uint2 *>(w.p2 + bi * 32 + 16 + 8 * h);
    b.m = *reinterpret_cast<const uint4 *>(w.p1 + bi * 16);
}
DEV void blk_load(Blk<FMT_IQ2S> &b, const PfMat &w, uint64_t bi, int) {
    const uint4 *p = reinterpret_cast<const uint4 *>(w.qs + bi * 64);
    b.g[0] = p[0]; b.g[1] = p[1]; b.sg[0] = p[2]; b.sg[1] = p[3];
    b.qh = *reinterpret_cast<const uint2 *>(w.p2 + bi * 8);
    b.sc = *reinterpret_cast<const uint2 *>(w.p1 + bi * 8);
    b.d = w.d[bi];
}
DEV void blk_load(Blk<FMT_IQ3S> &b, const PfMat &w, uint64_t bi, int) {
    const uint4 *p = reinterpret_cast<const uint4 *>(w.qs + bi * 64);
    b.q[0] = p[0]; b.q[1] = p[1]; b.q[2] = p[2]; b.q[3] = p[3];
    const uint4 *g = reinterpret_cast<const uint4 *>(w.p1 + bi * 32);
    b.sg[0] = g[0]; b.sg[1] = g[1];
    b.hs = *reinterpret_cast<const uint4 *>(w.p2 + bi * 16);
    b.d = w.d[bi];
}
DEV uint32_t byte_of(const uint4 (&v)[2], uint32_t i) { return (comp(v[i >> 4], (i >> 2) & 3) >> (8 * (i & 3))) & 255u; }
DEV uint32_t byte_of4(const uint4 (&v)[4], uint32_t i) { return (comp(v[i >> 4], (i >> 2) & 3) >> (8 * (i & 3))) & 255u; }

// B fragment of k-step s (8 fp16 codes).  IQ2_XS (src/qx_format.c:1914-1933): element
// 32ib+8l+j = db(l<2 ? lo : hi nibble of scales[ib]) * grid[q&511][j] * sign, q = qs[4ib+l];
// k-step s = 2ib + l/2, so q = qs[2s + h] and the nibble is s&1.
DEV uint4 frag(const Blk<FMT_IQ2> &b, int s, int h, const uint4 *G2, const uint4 *SG, const uint32_t *) {
    const uint32_t q = (comp(b.q[s >> 2], s & 3) >> (16 * h)) & 0xffffu;
    const uint32_t scb = ((s >> 1) < 4 ? b.sc.x : b.sc.y) >> (8 * ((s >> 1) & 3));
    const uint32_t nib = (scb >> (4 * (s & 1))) & 15u;
    uint4 g = G2[q & 511u];
    const uint4 m = SG[q >> 9];
    g.x ^= m.x; g.y ^= m.y; g.z ^= m.z; g.w ^= m.w;
    return hmul8(g, 2u * nib + 1u);
}
// IQ3_XXS (src/qx_format.c:1935-1959): element 32ib+8l+j (j<4) from grid3[qs[8ib+2l]],
// j>=4 from grid3[qs[8ib+2l+1]], signs ksigns[(aux[ib] >> 7l) & 127], scale
// d*(2(aux>>28)+1)/4; k-step s = 2ib + l/2.
DEV uint4 frag(const Blk<FMT_IQ3> &b, int s, int h, const uint4 *, const uint4 *SG, const uint32_t *G3) {
    const int ib = s >> 1, l = 2 * (s & 1) + h;
    const uint32_t dw = comp(b.q[ib >> 1], (2 * ib + (s & 1)) & 3) >> (16 * h);
    const uint32_t aux = comp(b.a[ib >> 2], ib & 3);
    const uint2 g1 = reinterpret_cast<const uint2 *>(G3)[dw & 255u];
    const uint2 g2 = reinterpret_cast<const uint2 *>(G3)[(dw >> 8) & 255u];
    const uint4 m = SG[(aux >> (7 * l)) & 127u];
    const uint4 g = make_uint4(g1.x ^ m.x, g1.y ^ m.y, g2.x ^ m.z, g2.y ^ m.w);
    return hmul8(g, 2u * (aux >> 28) + 1u);
}
// IQ4_XS (src/qx_format.c:2032-2053): element 32ib+j = kvalue[qs[16ib+j] & 15],
// 32ib+16+j = kvalue[qs[16ib+j] >> 4]; k-step 2ib takes the low nibbles of the lane's
// 8 bytes, 2ib+1 the high nibbles.
DEV uint4 frag(const Blk<FMT_IQ4> &b, int s, int, const uint4 *, const uint4 *, const uint32_t *KV2) {
    const uint2 q = b.q[s >> 1];
    uint32_t p[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[j] = KV2[(q.x >> (8 * j)) & 255u];
        p[4 + j] = KV2[(q.y >> (8 * j)) & 255u];
    }
    const uint32_t sel = (s & 1) ? 0x07060302u : 0x05040100u;
    return make_uint4(perm(p[1], p[0], sel), perm(p[3], p[2], sel), perm(p[5], p[4], sel), perm(p[7], p[6], sel));
}
// Q5_K (src/qx_format.c:2112-2145): element 32ib+l has the 5-bit code (nibble ib&1 of
// qs[32(ib/2)+l]) | (bit ib of qh[l]) << 4 and w = d*sc*code - dmin*m; k-step s = 2ib + t
// takes l = 16t + 8h + j.  Codes 0..31 go to fp16 exactly as bits(1024 + c) - 1024.
DEV uint32_t u8pair_h2(uint32_t w4, bool hi) {
    const h2v v = __builtin_bit_cast(h2v, perm(0u, w4, hi ? 0x0c030c02u : 0x0c010c00u) | 0x64006400u);
    const h2v k = {(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_bit_cast(uint32_t, v - k);
}
DEV uint4 frag(const Blk<FMT_Q5> &b, int s, int, const uint4 *, const uint4 *, const uint32_t *) {
    const int ib = s >> 1, t = s & 1;
    const uint2 q = b.q[2 * (ib >> 1) + t], qh = b.qh[t];
    const uint32_t nsh = 4 * (ib & 1);
    const uint32_t c0 = ((q.x >> nsh) & 0x0f0f0f0fu) | (((qh.x >> ib) & 0x01010101u) << 4);
    const uint32_t c1 = ((q.y >> nsh) & 0x0f0f0f0fu) | (((qh.y >> ib) & 0x01010101u) << 4);
    return make_uint4(u8pair_h2(c0, false), u8pair_h2(c0, true), u8pair_h2(c1, false), u8pair_h2(c1, true));
}
// IQ2_S (src/qx_format.c:1961-1984): entry e = 4ib + l (l = 2t + h) of the block: grid
// index qs[e] | ((qh[ib] >> 2l) & 3) << 8, explicit sign byte qs[32 + e], halves scaled by
// the nibble t of scales[ib] as IQ2_XS.
DEV uint4 frag(const Blk<FMT_IQ2S> &b, int s, int h, const uint4 *G2S, const uint4 *SG8, const uint32_t *) {
    const int ib = s >> 1, t = s & 1, l = 2 * t + h;
    const uint32_t e = 4 * ib + l;
    const uint32_t qh = ((ib < 4 ? b.qh.x : b.qh.y) >> (8 * (ib & 3))) & 255u;
    const uint32_t idx = byte_of(b.g, e) | (((qh >> (2 * l)) & 3u) << 8);
    uint4 g = G2S[idx];
    const uint4 m = SG8[byte_of(b.sg, e)];
    g.x ^= m.x; g.y ^= m.y; g.z ^= m.z; g.w ^= m.w;
    const uint32_t scb = ((ib < 4 ? b.sc.x : b.sc.y) >> (8 * (ib & 3))) & 255u;
    return hmul8(g, 2u * ((scb >> (4 * t)) & 15u) + 1u);
}
// IQ3_S (src/qx_format.c:1986-2030): k-step s = 2ib + t, lane half h: grid entries
// e = 8ib + 4t + 2h + {0, 1} (4 values each), index qs[e] | (bit e%8 of qh[ib]) << 8, sign
// byte signs[4ib + 2t + h], scale d*(2 sc + 1), sc the nibble ib&1 of scales[ib/2].
DEV uint4 frag(const Blk<FMT_IQ3S> &b, int s, int h, const uint4 *, const uint4 *SG8, const uint32_t *G3S) {
    const int ib = s >> 1, t = s & 1;
    const uint32_t e = 8 * ib + 4 * t + 2 * h;
    const uint32_t qh = (comp(b.hs, ib >> 2) >> (8 * (ib & 3))) & 255u;
    const uint32_t i1 = byte_of4(b.q, e) | (((qh >> (e & 7)) & 1u) << 8);
    const uint32_t i2 = byte_of4(b.q, e + 1) | (((qh >> ((e + 1) & 7)) & 1u) << 8);
    const uint2 g1 = reinterpret_cast<const uint2 *>(G3S)[i1];
    const uint2 g2 = reinterpret_cast<const uint2 *>(G3S)[i2];
    const uint4 m = SG8[byte_of(b.sg, 4 * ib + 2 * t + h)];
    const uint4 g = make_uint4(g1.x ^ m.x, g1.y ^ m.y, g2.x ^ m.z, g2.y ^ m.w);
    const uint32_t scw = (b.hs.z >> (8 * (ib >> 1))) & 255u;
    return hmul8(g, 2u * ((scw >> (4 * (ib & 1))) & 15u) + 1u);
}

// f32 scale of the partial sums: the block's d/8 or d/4; IQ4_XS: group ib's d*(ls-32)
DEV float blk_scale(const Blk<FMT_IQ2> &b, int) { return fp16_exact(b.d) * 0.125f; }
DEV float blk_scale(const Blk<FMT_IQ3> &b, int) { return fp16_exact(b.d) * 0.25f; }
DEV float blk_scale(const Blk<FMT_IQ4> &b, int ib) {
    const uint32_t sh = b.m.x >> 16, sl = (b.m.y >> (8 * (ib >> 1))) & 255u;
    const int ls = (int)(((sl >> (4 * (ib & 1))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
    return fp16_exact(b.m.x & 0xffffu) * (float)(ls - 32);
}
DEV float blk_scale(const Blk<FMT_IQ2S> &b, int) { return fp16_exact(b.d) * 0.125f; }
DEV float blk_scale(const Blk<FMT_IQ3S> &b, int) { return fp16_exact(b.d); }
// Q5_K sub-block ib: scale d*sc and offset dmin*m (6-bit sc, m: get_scale_min_k4,
// src/qx_format.c:2079-2087); meta = {d, dmin, scales[12]}
DEV uint32_t q5_scale_byte(const uint4 &m, int i) { return (comp(m, 1 + (i >> 2)) >> (8 * (i & 3))) & 255u; }
DEV void q5_sc_m(const Blk<FMT_Q5> &b, int ib, uint32_t &sc, uint32_t &mn) {
    if (ib < 4) {
        sc = q5_scale_byte(b.m, ib) & 63u;
        mn = q5_scale_byte(b.m, ib + 4) & 63u;
    } else {
        sc = (q5_scale_byte(b.m, ib + 4) & 15u) | ((q5_scale_byte(b.m, ib - 4) >> 6) << 4);
        mn = (q5_scale_byte(b.m, ib + 4) >> 4) | ((q5_scale_byte(b.m, ib) >> 6) << 4);
    }
}
DEV float blk_scale(const Blk<FMT_Q5> &b, int ib) {
    uint32_t sc, mn;
    q5_sc_m(b, ib, sc, mn);
    return fp16_exact(b.m.x & 0xffffu) * (float)sc;
}
template <int F> DEV float blk_offset(const Blk<F> &, int) { return 0.0f; }
DEV float blk_offset(const Blk<FMT_Q5> &b, int ib) {
    uint32_t sc, mn;
    q5_sc_m(b, ib, sc, mn);
    return fp16_exact(b.m.x >> 16) * (float)mn;
}

DEV f16x zero16() {
    f16x z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}
}  // namespace

// ================================================================= GEMM
// One wave: NSUB column tiles of 32 weight rows x NM row tiles of 32 tokens/slots, over
// all of K.  GU: the two column tiles are gate and up at the same rows (SwiGLU epilogue).
// Workgroup = 4 waves on 4 consecutive column tiles of the same row tiles.  The row
// tiles' fragments of one 256-value block (32 KiB per row tile) are copied by the whole
// workgroup into one of two LDS stages while the previous block is multiplied, and the
// next block's weights are loaded into registers at the same time, so each block's
// loads have one block of matrix work to arrive.  The loop has no data-dependent
// branches: the last iteration re-loads the last block (never used).
struct GemmLds {
    uint4 *g2, *sg, *a;   // a: two stages of `stage` uint4 each
    uint32_t *t;
    uint32_t stage;
};

// A fragments of block kb of NM row tiles: thread tid holds uint4 tid + 256*i (i < 8),
// kept in native 4-dword vectors (register-promoted; the uint4 struct array is not)
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
template <int NM>
DEV void a_load(v4u (&ra)[NM * 8], const uint4 *A, uint32_t KS, uint32_t kb) {
    const v4u *a = reinterpret_cast<const v4u *>(A);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) ra[m * 8 + i] = a[((uint64_t)m * KS + kb * 16) * 128 + 256 * i];
}
template <int NM>
DEV void a_store(const v4u (&ra)[NM * 8], uint4 *stage, int tid) {
    v4u *st = reinterpret_cast<v4u *>(stage);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) st[m * 2048 + tid + 256 * i] = ra[m * 8 + i];
}

// the 16 k-steps of one block: partial sums per block (IQ2_XS, IQ3_XXS) or per group of
// two k-steps (IQ4_XS), each scaled once into acc
template <int F, int NSUB, int NM>
DEV void block_mma(const Blk<F> (&bk)[NSUB], const uint4 *sa, f16x (&acc)[NSUB][NM], const GemmLds &L, int h,
                   int lane) {
    constexpr bool PER32 = F == FMT_IQ4 || F == FMT_Q5;   // a scale per 32-value group
    constexpr int NG = PER32 ? 8 : 1;
    float scl[NSUB][NG], ofs[NSUB][NG];
#pragma unroll
    for (int n = 0; n < NSUB; ++n)
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            scl[n][q] = blk_scale(bk[n], q);
            ofs[n][q] = F == FMT_Q5 ? blk_offset(bk[n], q) : 0.0f;
        }
    f16x G[NSUB][NM];
    f16x S[NM];   // Q5_K: sums of the activations over the group (B = all ones), for the dmin term
#pragma unroll
    for (int n = 0; n < NSUB; ++n)
#pragma unroll
        for (int m = 0; m < NM; ++m) G[n][m] = zero16();
#pragma unroll
    for (int m = 0; m < NM; ++m) S[m] = zero16();
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        uint4 ah[NM], al[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            ah[m] = sa[m * 2048 + s * 128 + lane];
            al[m] = sa[m * 2048 + s * 128 + 64 + lane];
        }
        if (F == FMT_Q5) {
            const uint4 ones = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);   // fp16 1.0
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                S[m] = mfma(ah[m], ones, S[m]);
                S[m] = mfma(al[m], ones, S[m]);
            }
        }
#pragma unroll
        for (int n = 0; n < NSUB; ++n) {
            const uint4 b = frag(bk[n], s, h, L.g2, L.sg, L.t);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                G[n][m] = mfma(ah[m], b, G[n][m]);
                G[n][m] = mfma(al[m], b, G[n][m]);
            }
        }
        if (PER32 && (s & 1)) {
#pragma unroll
            for (int n = 0; n < NSUB; ++n)
#pragma unroll
                for (int m = 0; m < NM; ++m) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[n][m][r] = fmaf(scl[n][s >> 1], G[n][m][r], acc[n][m][r]);
                        if (F == FMT_Q5) acc[n][m][r] = fmaf(-ofs[n][s >> 1], S[m][r], acc[n][m][r]);
                    }
                    G[n][m] = zero16();
                }
            if (F == FMT_Q5)
#pragma unroll
                for (int m = 0; m < NM; ++m) S[m] = zero16();
        }
        // LDS reads of later k-steps stay behind this point: the unrolled loop would
        // otherwise hoist all of them into registers
        if (s & 1) asm volatile("" ::: "memory");
    }
    if (!PER32) {
#pragma unroll
        for (int n = 0; n < NSUB; ++n)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][m][r] = fmaf(scl[n][0], G[n][m][r], acc[n][m][r]);
    }
}

template <int F, int NSUB, int NM, int EPI>
DEV void gemm_body(const PfGemm &g, const GemmLds &L, uint32_t e, uint32_t mt0, uint32_t bx) {
    constexpr bool GU = EPI == EPI_SWIGLU;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), h = lane >> 5, col = lane & 31;
    const uint32_t KB = g.kb, KS = 16 * KB;
    const uint32_t nt = bx * 4 + wave;                    // column tile group of this wave
    const uint32_t c0 = GU ? 32 * nt : 32 * NSUB * nt;     // first output column
    PfMat W[NSUB];
    uint64_t rowblk[NSUB];
#pragma unroll
    for (int n = 0; n < NSUB; ++n) {
        const uint32_t c = GU ? c0 : c0 + 32 * n;
        const int mi = GU ? n : (c >= g.w_start[2] ? 2 : c >= g.w_start[1] ? 1 : 0);
        W[n] = g.w[mi];
        const uint32_t r = (GU ? c0 : c - g.w_start[mi]) + col;
        rowblk[n] = ((uint64_t)e * g.rows + r) * KB;
    }
    const uint4 *A = g.apk + (uint64_t)mt0 * KS * 128 + tid;
    uint4 *stage0 = L.a, *stage1 = L.a + L.stage;

    f16x acc[NSUB][NM];
#pragma unroll
    for (int n = 0; n < NSUB; ++n)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[n][m] = zero16();
    // weights of even blocks in b0, odd blocks in b1; A of block kb in stage kb&1
    Blk<F> b0[NSUB], b1[NSUB];
    v4u ra[NM * 8];
    const uint32_t k1 = KB > 1 ? 1 : 0;
#pragma unroll
    for (int n = 0; n < NSUB; ++n) blk_load(b0[n], W[n], rowblk[n], h);
    a_load<NM>(ra, A, KS, 0);
    a_store<NM>(ra, stage0, tid);
    a_load<NM>(ra, A, KS, k1);
#pragma unroll
    for (int n = 0; n < NSUB; ++n) blk_load(b1[n], W[n], rowblk[n] + k1, h);
    __syncthreads();   // tables and stage 0

    // per block: multiply, stage the next block's A (its stage was last read two blocks
    // back, before the barrier that ended the previous block), then start the loads of
    // the block after it (clamped to the last block: always in bounds, never used)
#pragma unroll 1
    for (uint32_t kb = 0; kb < KB; kb += 2) {
        block_mma<F, NSUB, NM>(b0, stage0, acc, L, h, lane);
        a_store<NM>(ra, stage1, tid);
        {
            const uint32_t kn = kb + 2 < KB ? kb + 2 : KB - 1;
            a_load<NM>(ra, A, KS, kn);
#pragma unroll
            for (int n = 0; n < NSUB; ++n) blk_load(b0[n], W[n], rowblk[n] + kn, h);
        }
        __syncthreads();
        if (kb + 1 >= KB) break;
        block_mma<F, NSUB, NM>(b1, stage1, acc, L, h, lane);
        a_store<NM>(ra, stage0, tid);
        {
            const uint32_t kn = kb + 3 < KB ? kb + 3 : KB - 1;
            a_load<NM>(ra, A, KS, kn);
#pragma unroll
            for (int n = 0; n < NSUB; ++n) blk_load(b1[n], W[n], rowblk[n] + kn, h);
        }
        __syncthreads();
    }

    // epilogue: lane's column c, rows 8*(r/4) + 4h + r%4 of each row tile
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint32_t rbase = (mt0 + m) * 32 + 4 * h;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = rbase + 8 * (r >> 2) + (r & 3);
            if (!g.mgroups && row >= g.nvalid) continue;
            const float rs = g.rscale[row];
            if (EPI == EPI_SWIGLU) {
                float gv = acc[0][m][r] * rs, uv = acc[1][m][r] * rs;
                gv = isfinite(gv) ? gv : 0.0f;
                uv = isfinite(uv) ? uv : 0.0f;
                // qx_silu (src/qx_format.c:2511-2513) in f32: relative error ~1e-7 against the
                // reference's double, far inside the 1e-5 bar; a double exp per output was a
                // large share of the epilogue
                const float sg = gv / (1.0f + expf(-gv));
                g.out[(uint64_t)row * g.ld + c0 + col] = sg * uv;
            } else {
#pragma unroll
                for (int n = 0; n < NSUB; ++n) {
                    const uint32_t c = c0 + 32 * n + col;
                    float y = acc[n][m][r] * rs;
                    y = isfinite(y) ? y : 0.0f;   // non-finite projection outputs -> 0 (src/qx_format.c:4284)
                    const uint64_t o = (uint64_t)row * g.ld + c;
                    if (EPI == EPI_RESID) {
                        if (g.dump) g.dump[o] = y;
                        g.out[o] = g.resid[o] + y;
                    } else {
                        g.out[o] = y;
                    }
                }
            }
        }
    }
}

// XCD-aware tile order.  Workgroups go to the 8 XCDs round-robin by linear index, and each
// XCD has its own L2, so a row tile's packed activations are fetched once into every L2
// whose XCD runs one of its column workgroups, and a weight column group once into every
// L2 that runs one of its row tiles.  Workgroup L (on XCD r = L % 8) takes the tile
// (x, y) with y % a == r / b and x % b == r % b, a = xcd_rows row classes, b = 8 / a column
// classes: each XCD then reads 1/a of the activations and 1/b of the weights.  The
// launcher makes gridDim.x a multiple of b and gridDim.y of a (extra rows return).
DEV void xcd_tile(uint32_t a, uint32_t &bx, uint32_t &by) {
    const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y, r = L & 7u, j = L >> 3;
    const uint32_t b = 8u / a, nxb = gridDim.x / b;
    bx = (j % nxb) * b + r % b;
    by = (j / nxb) * a + r / b;
}

template <int F, int NSUB, int MT, int EPI>
__global__ __launch_bounds__(256, MT == 1 && F != FMT_IQ2S ? 2 : 1) void qxp_gemm(PfGemm g, PfTables P) {   // (IQ2_S: 86 KB of LDS, one per CU)
    uint32_t e = 0, mt0, nmt, bx, by;
    xcd_tile(g.xcd_rows, bx, by);
    if (g.mgroups) {
        if (by >= g.meta[0]) return;   // whole workgroup
        const uint32_t mg = g.mgroups[by];
        e = mg & 255u; mt0 = (mg >> 8) & 0xfffu; nmt = mg >> 20;
    } else {
        mt0 = by * MT;
        if (mt0 >= g.mtiles) return;   // whole workgroup: a padding row
        nmt = min((uint32_t)MT, g.mtiles - mt0);
    }
    constexpr int NG2 = F == FMT_IQ2 ? 512 : F == FMT_IQ2S ? 1024 : 1;        // fp16 grid entries of 8
    constexpr int NSG = F == FMT_IQ2 || F == FMT_IQ3 ? 128 : F == FMT_IQ2S || F == FMT_IQ3S ? 256 : 1;   // sign masks
    constexpr int NT4 = F == FMT_IQ3 ? 512 : F == FMT_IQ3S ? 1024 : F == FMT_IQ4 ? 256 : 1;   // words
    __shared__ uint4 s_g2[NG2];
    __shared__ uint4 s_sg[NSG];
    __shared__ uint32_t s_t[NT4];
    __shared__ uint4 s_a[2 * MT * 2048];   // [stage][row tile][(kstep*2 + piece)*64 + lane]
    const int tid = threadIdx.x;
    {
        const uint4 *g2 = F == FMT_IQ2S ? P.g2sh : P.g2h;
        const uint4 *sg = F == FMT_IQ2S || F == FMT_IQ3S ? P.sgn8 : P.sgn;
        const uint32_t *t4 = F == FMT_IQ3 ? reinterpret_cast<const uint32_t *>(P.g3h)
                           : F == FMT_IQ3S ? reinterpret_cast<const uint32_t *>(P.g3sh) : P.kv2;
        if (NG2 > 1) for (int i = tid; i < NG2; i += 256) s_g2[i] = g2[i];
        if (NSG > 1) for (int i = tid; i < NSG; i += 256) s_sg[i] = sg[i];
        if (NT4 > 1) for (int i = tid; i < NT4; i += 256) s_t[i] = t4[i];
    }
    const GemmLds L{s_g2, s_sg, s_a, s_t, MT * 2048};
    if (MT == 2 && nmt == 2) gemm_body<F, NSUB, (MT == 2 ? 2 : 1), EPI>(g, L, e, mt0, bx);
    else gemm_body<F, NSUB, 1, EPI>(g, L, e, mt0, bx);
}

// ================================================================= element-wise stages
// Q4_K embedding rows of tokens[0..T) (src/qx_format.c:3759-3793); block per token.
extern "C" __global__ __launch_bounds__(256) void qxp_embed(const uint8_t *emb, uint64_t row_bytes,
                                                            const uint32_t *tokens, float *x) {
    embed_q4k_row(emb + (uint64_t)tokens[blockIdx.x] * row_bytes, x + (uint64_t)blockIdx.x * 2048);
}

// RMSNorm of each token's 2048-vector (qx_apply_f32_rmsnorm, src/qx_format.c:3358-3371);
// wave per token.
extern "C" __global__ __launch_bounds__(256) void qxp_norm(const float *x, const float *w, uint32_t T, float *y) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + wave_id();
    if (t >= T) return;
    float v[32], ww[32];
    load32(x + (uint64_t)t * 2048 + 32 * lane, v);
    load32(w + 32 * lane, ww);
    rmsnorm32(v, ww);
    float4 *o = reinterpret_cast<float4 *>(y + (uint64_t)t * 2048 + 32 * lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

// Packs one row of the A operand held by a wave, NC chunks of 8 values per lane (chunk
// index c[i]): scaled by a power of two and split into fp16 hi/lo fragments; rscale[r]
// = 1/s, or 0 (and zeros) when the row has a non-finite value.
template <int NC, int K>
DEV void pack_row(const float (&v)[NC][8], const int (&c)[NC], uint32_t r, uint4 *apk, float *rscale) {
    constexpr int CH = K / 8, KS = K / 16;
    const int lane = threadIdx.x & 63;
    float mx = 0.0f;
    bool fin = true;
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            fin = fin && isfinite(v[i][j]);
            mx = fmaxf(mx, fabsf(v[i][j]));
        }
    const bool ok = __ballot(!fin) == 0;
    mx = fmaxf(mx, dppf<DPP_XOR1>(mx)); mx = fmaxf(mx, dppf<DPP_XOR2>(mx));
    mx = fmaxf(mx, dppf<DPP_ROR4>(mx)); mx = fmaxf(mx, dppf<DPP_ROR8>(mx));
    mx = fmaxf(fmaxf(rdlanef(mx, 0), rdlanef(mx, 16)), fmaxf(rdlanef(mx, 32), rdlanef(mx, 48)));
    int ex = 0;
    if (mx > 0.0f && ok) (void)frexpf(mx, &ex);   // mx = f * 2^ex, f in [0.5, 1)
    int sh = 14 - ex;
    sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
    const float sc = ldexpf(1.0f, sh);
    if (lane == 0) rscale[r] = ok ? ldexpf(1.0f, -sh) : 0.0f;
    const uint32_t mt = r >> 5, i32 = r & 31;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        if (c[i] >= CH) continue;
        h8v hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float y = ok ? v[i][j] * sc : 0.0f;
            const _Float16 a = (_Float16)y;
            hi[j] = a;
            lo[j] = (_Float16)(y - (float)a);
        }
        const uint64_t base = ((uint64_t)mt * KS + (c[i] >> 1)) * 128 + i32 + 32 * (c[i] & 1);
        apk[base] = __builtin_bit_cast(uint4, hi);
        apk[base + 64] = __builtin_bit_cast(uint4, lo);
    }
}

// Packs row r of the A operand (r < rows, and r < nrows[1] when nrows is non-null):
// source row map ? map[r] : r of src (K floats; rows r >= nvalid and negative map
// entries are padding and pack zeros), through pack_row.  Wave per row, chunks
// lane + 64 i, no workgroup barriers.
template <int K>
__global__ __launch_bounds__(256) void qxp_pack(const float *src, const int32_t *map, const uint32_t *nrows,
                                                uint32_t rows, uint32_t nvalid, uint4 *apk, float *rscale) {
    constexpr int CH = K / 8, PL = (CH + 63) / 64;
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * 4 + wave_id();
    if (r >= rows || (nrows && r >= nrows[1])) return;   // whole wave
    const int32_t sr = r >= nvalid ? -1 : map ? map[r] : (int32_t)r;
    float v[PL][8];
    int c[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        c[i] = lane + 64 * i;
        if (c[i] < CH && sr >= 0) {
            const float4 *p = reinterpret_cast<const float4 *>(src + (uint64_t)sr * K + 8 * c[i]);
            const float4 a = p[0], b = p[1];
            v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
            v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
        }
    }
    pack_row<PL, K>(v, c, r, apk, rscale);
}

// RMSNorm of token r (qxp_norm's arithmetic: 32 consecutive values per lane) fused with
// its packing as the Q/K/V GEMM's A operand; rows r >= nvalid pack zeros.
extern "C" __global__ __launch_bounds__(256) void qxp_norm_pack(const float *x, const float *w, uint32_t rows,
                                                                uint32_t nvalid, uint4 *apk, float *rscale) {
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * 4 + wave_id();
    if (r >= rows) return;   // whole wave
    float v[4][8];
    const int c[4] = {4 * lane, 4 * lane + 1, 4 * lane + 2, 4 * lane + 3};
    if (r < nvalid) {
        float t[32], ww[32];
        load32(x + (uint64_t)r * 2048 + 32 * lane, t);
        load32(w + 32 * lane, ww);
        rmsnorm32(t, ww);
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i >> 3][i & 7] = t[i];
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i >> 3][i & 7] = 0.0f;
    }
    pack_row<4, 2048>(v, c, r, apk, rscale);
}

// Per token (block): q/k head RMSNorm (src/qx_format.c:3740-3757) and RoPE at position
// p0+t (4625-4641), INT8 quantization of K and V over all 512 values (4449-4463) into
// the cache row [layer][p0+t]; the roped q (f32) goes to qr for attention.
extern "C" __global__ __launch_bounds__(256) void qxp_qk(const float *qkv, const float *q_norm, const float *k_norm,
        Tables T, int8_t *kc, int8_t *vc, float *ks, float *vs, uint32_t layer, uint32_t ctx, uint32_t p0, float *qr) {
    __shared__ float s_k[512], s_v[512];
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t t = blockIdx.x, pos = p0 + t;
    const float *row = qkv + (uint64_t)t * 5120;
    float k0 = row[4096 + 128 * wave + lane], k1 = row[4096 + 128 * wave + 64 + lane];
    const float v0 = row[4608 + tid], v1 = row[4608 + 256 + tid];
    const float kw0 = k_norm[lane], kw1 = k_norm[64 + lane], qw0 = q_norm[lane], qw1 = q_norm[64 + lane];
    const double c = T.rope_cos[pos * 64 + lane], s = T.rope_sin[pos * 64 + lane];
    head_norm_rope_wave(k0, k1, kw0, kw1, c, s);
    s_k[128 * wave + lane] = k0;
    s_k[128 * wave + 64 + lane] = k1;
    s_v[tid] = v0;
    s_v[256 + tid] = v1;
#pragma unroll 1
    for (int hh = 0; hh < 8; ++hh) {
        const int qh = 8 * wave + hh;
        float q0 = row[128 * qh + lane], q1 = row[128 * qh + 64 + lane];
        head_norm_rope_wave(q0, q1, qw0, qw1, c, s);
        qr[(uint64_t)t * 4096 + 128 * qh + lane] = q0;
        qr[(uint64_t)t * 4096 + 128 * qh + 64 + lane] = q1;
    }
    float ka = fmaxf(int8_mag(k0), int8_mag(k1)), va = fmaxf(int8_mag(v0), int8_mag(v1));
    ka = block_max256(ka, red);
    va = block_max256(va, red);
    const float kscale = int8_scale(ka), vscale = int8_scale(va);
    const uint64_t slot = (uint64_t)layer * ctx + pos;
    for (int i = tid; i < 512; i += 256) {
        kc[slot * 512 + i] = int8_code(s_k[i], kscale);
        vc[slot * 512 + i] = int8_code(s_v[i], vscale);
    }
    if (tid == 0) { ks[slot] = kscale; vs[slot] = vscale; }
}

// Causal GQA attention of the chunk on the matrix cores (qx_rope_gqa_attention_partial,
// src/qx_format.c:5051-5196, for every token of the chunk at once).  A workgroup takes
// one KV head and 4 consecutive tokens: the 8 q heads of the KV head x 4 tokens are the
// 32 columns of v_mfma_f32_32x32x16_f16 (column c: head c/4, token c%4).  Its 4 waves
// take the 32-position chunks ci = wave, wave+4, ... of positions 0..p0+t and keep, per
// column, a running maximum, denominator and context (online softmax; the reference
// normalises with the global maximum, the same quantity up to rounding).  Per chunk:
//   scores  S^T[pos][col] = K8[pos][:] . q[col][:]: A = the chunk's INT8 K codes
//           (exact in fp16), B = q split hi + lo in fp16 after a power-of-two row
//           scale (max |q| in [2^13, 2^14)); f32 accumulation; times ks[pos] /
//           sqrt(128) and the row scale; positions past the token masked;
//   weights p = exp(s - m) (f32), pv = p * vs[pos], split hi + lo after a power-of-two
//           scale per column and chunk;
//   context C[dim][col] += V8^T[dim][pos] . pv[pos][col] (A = V codes from a transposed
//           LDS copy of the chunk), rescaled by exp(m_old - m_new) per column.
// The result registers of the score product are exactly the k layout the context
// product's B operand needs (lane l: column l%32, positions 8(r/4) + 4(l/32) + r%4 of
// register r), so the weights never leave the lane.  The waves' states are merged in
// LDS at the end and the context is divided by the denominator.
namespace {
constexpr int PA_TT = 4;   // tokens per workgroup

DEV uint4 i8x8_to_f16(uint2 v) {   // 8 int8 -> 8 exact fp16 (bias 0x64 trick: 1024 + (b ^ 0x80) - 1152)
    const h2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t x = v.x ^ 0x80808080u, y = v.y ^ 0x80808080u;
    const uint32_t c = 0x64646464u;
    auto cv = [&](uint32_t w) { return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, w) - bias); };
    return make_uint4(cv(perm(c, x, 0x04010400u)), cv(perm(c, x, 0x04030402u)), cv(perm(c, y, 0x04010400u)),
                      cv(perm(c, y, 0x04030402u)));
}
DEV void split8(const float (&v)[8], float sc, uint4 &hi, uint4 &lo) {   // v * sc = hi + lo (+ 2^-22 rel)
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = v[2 * i] * sc, b = v[2 * i + 1] * sc;
        const _Float16 ha = (_Float16)a, hb = (_Float16)b;
        const _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
        const h2v hh = {ha, hb}, ll = {la, lb};
        h[i] = __builtin_bit_cast(uint32_t, hh);
        l[i] = __builtin_bit_cast(uint32_t, ll);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}
DEV float pow2_scale(float mx) {   // 2^(14-e) with mx = m * 2^e, m in [0.5, 1): mx * scale in [2^13, 2^14)
    int e = 0;
    if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &e);
    return mx > 0.0f && isfinite(mx) ? ldexpf(1.0f, 14 - e) : 1.0f;
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void qxp_attn(const float *qr, const int8_t *kc, const int8_t *vc,
        const float *ks, const float *vs, uint32_t layer, uint32_t ctx, uint32_t p0, uint32_t T, float *ctx_out) {
    __shared__ uint32_t s_vt[4][128 * 9];   // per wave: V^T of its chunk, rows of 36 bytes (32 positions)
    __shared__ float s_ks[4][32], s_vs[4][32];
    __shared__ float s_acc[2][32][129];
    __shared__ float s_m[2][32], s_den[2][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, h = lane >> 5;
    const uint32_t kh = blockIdx.x, t0 = blockIdx.y * PA_TT;
    const uint32_t tt = t0 + (col & 3), qh = kh * 8 + (col >> 2);
    const bool tok_ok = tt < T;
    const uint32_t limit = p0 + (tok_ok ? tt : 0);              // last position of the column's token
    const uint32_t last_t = min(t0 + PA_TT, T) - 1;
    const uint32_t npos = p0 + last_t + 1;                      // positions the workgroup needs
    const uint64_t base = (uint64_t)layer * ctx;
    // q fragments: k-step s holds dims 16s + 8h + j of the column's q row
    float qv[8][8];
    bool fin = true;
    float qmx = 0.0f;
    const float *qrow = qr + (uint64_t)(tok_ok ? tt : 0) * 4096 + qh * 128 + 8 * h;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
        const float4 a = *reinterpret_cast<const float4 *>(qrow + 16 * s8);
        const float4 b = *reinterpret_cast<const float4 *>(qrow + 16 * s8 + 4);
        qv[s8][0] = a.x; qv[s8][1] = a.y; qv[s8][2] = a.z; qv[s8][3] = a.w;
        qv[s8][4] = b.x; qv[s8][5] = b.y; qv[s8][6] = b.z; qv[s8][7] = b.w;
#pragma unroll
        for (int j = 0; j < 8; ++j) { fin = fin && isfinite(qv[s8][j]); qmx = fmaxf(qmx, fabsf(qv[s8][j])); }
    }
    fin = fin && (__shfl_xor((int)fin, 32) != 0);
    qmx = fmaxf(qmx, __shfl_xor(qmx, 32));
    // a non-finite q makes every score non-finite, which the reference stores as 0
    const bool qz = !fin || !tok_ok;
    const float qsc = pow2_scale(qz ? 0.0f : qmx);
    uint4 qhi[8], qlo[8];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
        if (qz) {
#pragma unroll
            for (int j = 0; j < 8; ++j) qv[s8][j] = 0.0f;
        }
        split8(qv[s8], qsc, qhi[s8], qlo[s8]);
    }
    const float sfac = (float)(1.0 / ((double)qsc * sqrt(128.0)));   // exact power of two over sqrt(128)
    float m_run = -INFINITY, den = 0.0f;
    f16x acc[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[d] = zero16();
    const uint32_t nchunk = (npos + 31) / 32;
    uint32_t *vt = s_vt[wave];
#pragma unroll 1
    for (uint32_t ci = wave; ci < nchunk; ci += 4) {
        const uint32_t pb = ci * 32;
        // K fragments of position pb + col (clamped inside the workgroup's range)
        const uint32_t pk = min(pb + col, npos - 1);
        const int8_t *krow = kc + (base + pk) * 512 + kh * 128 + 8 * h;
        uint2 kq[8];
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) kq[s8] = *reinterpret_cast<const uint2 *>(krow + 16 * s8);
        if (lane < 32) {
            const uint32_t pp = min(pb + lane, npos - 1);
            s_ks[wave][lane] = ks[base + pp];
            s_vs[wave][lane] = vs[base + pp];
        }
        // V^T of the chunk: lane takes 4 blocks of 4 positions x 4 dims and transposes them
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bq = lane + 64 * i, pq = bq & 7, dq = bq >> 3;
            uint32_t w[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t pp = min(pb + 4 * pq + r, npos - 1);
                w[r] = *reinterpret_cast<const uint32_t *>(vc + (base + pp) * 512 + kh * 128 + 4 * dq);
            }
            const uint32_t a0 = perm(w[1], w[0], 0x05010400u), a1 = perm(w[3], w[2], 0x05010400u);
            const uint32_t a2 = perm(w[1], w[0], 0x07030602u), a3 = perm(w[3], w[2], 0x07030602u);
            vt[(4 * dq + 0) * 9 + pq] = perm(a1, a0, 0x05040100u);
            vt[(4 * dq + 1) * 9 + pq] = perm(a1, a0, 0x07060302u);
            vt[(4 * dq + 2) * 9 + pq] = perm(a3, a2, 0x05040100u);
            vt[(4 * dq + 3) * 9 + pq] = perm(a3, a2, 0x07060302u);
        }
        // scores: S^T = K8 . q
        f16x sacc = zero16();
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            const uint4 kf = i8x8_to_f16(kq[s8]);
            sacc = mfma(kf, qhi[s8], sacc);
            sacc = mfma(kf, qlo[s8], sacc);
        }
        // register r: position pb + 8(r/4) + 4h + r%4
        float sc[16], cmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t pr = 8 * (r >> 2) + 4 * h + (r & 3), p = pb + pr;
            float v = sacc[r] * (s_ks[wave][pr] * sfac);
            v = isfinite(v) ? v : 0.0f;
            sc[r] = p <= limit ? v : -INFINITY;
            cmax = fmaxf(cmax, sc[r]);
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = m_new == -INFINITY ? 1.0f : __expf(m_run - m_new);
        float pv[16], psum = 0.0f, pmx = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t pr = 8 * (r >> 2) + 4 * h + (r & 3);
            const float e = sc[r] == -INFINITY ? 0.0f : __expf(sc[r] - m_new);
            psum += e;
            pv[r] = e * s_vs[wave][pr];
            pmx = fmaxf(pmx, pv[r]);
        }
        pmx = fmaxf(pmx, __shfl_xor(pmx, 32));
        den = den * alpha + psum;
        m_run = m_new;
        const float psc = pow2_scale(pmx), pinv = 1.0f / psc;   // powers of two: exact
        uint4 phi[2], plo[2];
        {
            float a8[8], b8[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) { a8[j] = pv[j]; b8[j] = pv[8 + j]; }
            split8(a8, psc, phi[0], plo[0]);
            split8(b8, psc, phi[1], plo[1]);
        }
        // context: per 32-dim tile, C[dim][col] = V8^T . pv, merged into the running sums
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            f16x cacc = zero16();
            const uint32_t *row = vt + (32 * d + col) * 9;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const uint4 vf = i8x8_to_f16(make_uint2(row[4 * s2 + h], row[4 * s2 + 2 + h]));
                cacc = mfma(vf, phi[s2], cacc);
                cacc = mfma(vf, plo[s2], cacc);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[d][r] = fmaf(acc[d][r], alpha, cacc[r] * pinv);
        }
    }
    // merge the 4 waves' (max, denominator, context) per column: 2+3 into 0+1, then 1 into 0
    den += __shfl_xor(den, 32);
#pragma unroll 1
    for (int round = 0; round < 2; ++round) {
        const int nw = round == 0 ? 2 : 1;   // waves [nw, 2nw) hand over to [0, nw)
        if (wave >= nw && wave < 2 * nw) {
            const int slot = wave - nw;
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) s_acc[slot][col][32 * d + 8 * (r >> 2) + 4 * h + (r & 3)] = acc[d][r];
            if (h == 0) { s_m[slot][col] = m_run; s_den[slot][col] = den; }
        }
        __syncthreads();
        if (wave < nw) {
            const float mo = s_m[wave][col], dn = s_den[wave][col];
            const float m_new = fmaxf(m_run, mo);
            const float fa = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
            const float fb = mo == -INFINITY ? 0.0f : __expf(mo - m_new);
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[d][r] = acc[d][r] * fa + s_acc[wave][col][32 * d + 8 * (r >> 2) + 4 * h + (r & 3)] * fb;
            den = den * fa + dn * fb;
            m_run = m_new;
        }
        __syncthreads();
    }
    if (wave == 0 && tok_ok) {
        const float inv = 1.0f / den;
        float *out = ctx_out + (uint64_t)tt * 4096 + qh * 128;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) out[32 * d + 8 * (r >> 2) + 4 * h + (r & 3)] = acc[d][r] * inv;
    }
}

// Router logits on the FP64 matrix cores: logit[t][e] = sum_i (double)W[e][i] *
// (double)xn[t][i] (src/qx_format.c:5254-5264: the same exact double products, summed in
// another order, within ~1e-15 relative of the reference's sequential sum; equal router
// rows still give equal logits).  A workgroup owns a 16 x 16 (token x expert) tile; its 8
// waves split K = 2048 in eighths and lane group g = lane / 16 of a wave feeds k-slot g
// of v_mfma_f64_16x16x4 with 64 consecutive k of the wave's 256.  The 8 partial tiles
// are added in LDS in a fixed order.
typedef double f64x4 __attribute__((ext_vector_type(4)));
extern "C" __global__ __launch_bounds__(512) void qxp_router(const float *xn, const float *router, uint32_t T,
                                                             uint32_t experts, double *logits) {
    __shared__ double part[8][16][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int i = lane & 15, g = lane >> 4;
    const uint32_t t = blockIdx.x * 16 + i;   // < 512: xn holds QXP_MAX rows
    const uint32_t e = blockIdx.y * 16 + i, er = e < experts ? e : 0u;
    const float4 *xa = reinterpret_cast<const float4 *>(xn + (uint64_t)t * 2048 + wave * 256 + g * 64);
    const float4 *wb = reinterpret_cast<const float4 *>(router + (uint64_t)er * 2048 + wave * 256 + g * 64);
    f64x4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 4
    for (int j = 0; j < 16; ++j) {
        const float4 a = xa[j], b = wb[j];
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.x, (double)b.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.y, (double)b.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.z, (double)b.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.w, (double)b.w, acc, 0, 0, 0);
    }
    // result r of lane l: token row l / 16 + 4 * r, expert column l % 16 (the f64 16x16
    // layout, unlike the f32 ones' 4 * (l / 16) + r)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][g + 4 * r][i] = acc[r];
    __syncthreads();
    if (tid < 256) {
        const int row = tid >> 4, col = tid & 15;
        const double v = ((part[0][row][col] + part[1][row][col]) + (part[2][row][col] + part[3][row][col])) +
                         ((part[4][row][col] + part[5][row][col]) + (part[6][row][col] + part[7][row][col]));
        const uint32_t tt = blockIdx.x * 16 + row, ee = blockIdx.y * 16 + col;
        if (tt < T && ee < experts) logits[(uint64_t)tt * 128 + ee] = v;
    }
}

// Top-8 experts and renormalised weights per token (wave per token; the decode path's
// selection, src/qx_format.c:5265-5285).
extern "C" __global__ __launch_bounds__(256) void qxp_route(const double *logits, uint32_t T, uint32_t experts,
                                                            uint32_t *ids, double *wts) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + wave_id();
    if (t >= T) return;
    const int E = (int)experts;
    const double l0 = lane < E ? logits[(uint64_t)t * 128 + lane] : 0.0;
    const double l1 = lane + 64 < E ? logits[(uint64_t)t * 128 + lane + 64] : 0.0;
    uint32_t id[QXG_TOPK];
    double w[QXG_TOPK];
    wave_top8(l0, l1, E, id, w);
#pragma unroll
    for (int q = 0; q < QXG_TOPK; ++q)
        if (lane == q) { ids[t * 8 + q] = id[q] < experts ? id[q] : 0u; wts[t * 8 + q] = w[q]; }
}

// Token -> expert grouping (one block): expert e's tokens, ascending, take slots
// off[e] .. off[e]+n_e of an expert-major layout padded to 32 per expert; tok_slot[t][r]
// is the slot of (token t, rank r), slot_token the inverse (-1 on padding).  m-groups of
// up to MT row tiles per expert feed the expert GEMMs; meta = {m-groups, padded slots}.
extern "C" __global__ __launch_bounds__(1024) void qxp_group(const uint32_t *ids, uint32_t T, uint32_t experts,
        uint32_t mt_per_group, int32_t *slot_token, uint32_t *tok_slot, uint32_t *mgroups, uint32_t *meta) {
    __shared__ uint32_t bm[128][QXP_MAX / 32];
    __shared__ uint32_t cnt[128], off[129];
    const int tid = threadIdx.x;
    for (int i = tid; i < 128 * (QXP_MAX / 32); i += 1024) (&bm[0][0])[i] = 0u;
    __syncthreads();
    for (uint32_t p = tid; p < T * 8; p += 1024) {
        const uint32_t t = p >> 3, e = ids[p];
        atomicOr(&bm[e][t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    if (tid < 128) {
        uint32_t c = 0;
        for (int w = 0; w < QXP_MAX / 32; ++w) c += __popc(bm[tid][w]);
        cnt[tid] = c;
    }
    __syncthreads();
    if (tid < 64) {   // wave 0: experts 2l, 2l+1 per lane; exclusive scans of row tiles and m-groups
        uint32_t mt[2], ng[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t e = 2 * tid + j;
            mt[j] = e < experts ? (cnt[e] + 31) / 32 : 0u;
            ng[j] = (mt[j] + mt_per_group - 1) / mt_per_group;
        }
        const uint32_t smt = mt[0] + mt[1], sng = ng[0] + ng[1];
        uint32_t imt = smt, ing = sng;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t a = __shfl_up(imt, o), b = __shfl_up(ing, o);
            if (tid >= o) { imt += a; ing += b; }
        }
        uint32_t tile = imt - smt, gi = ing - sng;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t e = 2 * tid + j;
            if (e <= 128u) off[e] = 32 * tile;
            for (uint32_t g = 0; g < mt[j]; g += mt_per_group) {
                const uint32_t k = mt[j] - g < mt_per_group ? mt[j] - g : mt_per_group;
                mgroups[gi++] = e | ((tile + g) << 8) | (k << 20);
            }
            tile += mt[j];
        }
        if (tid == 63) {   // totals (experts past `experts` hold no tiles)
            off[experts] = 32 * imt;
            meta[0] = ing;
            meta[1] = 32 * imt;
        }
    }
    __syncthreads();
    for (uint32_t p = tid; p < T * 8; p += 1024) {
        const uint32_t t = p >> 3, e = ids[p], w = t >> 5;
        uint32_t rank = __popc(bm[e][w] & ((1u << (t & 31)) - 1u));
        for (uint32_t i = 0; i < w; ++i) rank += __popc(bm[e][i]);
        const uint32_t slot = off[e] + rank;
        tok_slot[p] = slot;
        slot_token[slot] = (int32_t)t;
    }
    if (tid < (int)experts)
        for (uint32_t s = off[tid] + cnt[tid]; s < off[tid + 1]; ++s) slot_token[s] = -1;
}

// x[t][i] = x1[t][i] + sum_r (float)(w_r * (double)y[slot(t,r)][i]), ranks in order
// (src/qx_format.c:5296-5309); block per token.
extern "C" __global__ __launch_bounds__(256) void qxp_combine(const float *x1, const float *y, const uint32_t *tok_slot,
                                                              const double *wts, float *x, float *moe_dump) {
    const uint32_t t = blockIdx.x;
    uint32_t sl[QXG_TOPK];
    double w[QXG_TOPK];
#pragma unroll
    for (int r = 0; r < QXG_TOPK; ++r) { sl[r] = tok_slot[t * 8 + r]; w[r] = wts[t * 8 + r]; }
    for (int i = threadIdx.x; i < 2048; i += 256) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < QXG_TOPK; ++r) m += (float)(w[r] * (double)y[(uint64_t)sl[r] * 2048 + i]);
        if (moe_dump) moe_dump[(uint64_t)t * 2048 + i] = m;
        x[(uint64_t)t * 2048 + i] = x1[(uint64_t)t * 2048 + i] + m;
    }
}

// ================================================================= launch wrappers
extern "C" {
void qxp_launch_gemm(hipStream_t s, int kind, const PfGemm &g0, const PfTables &P, uint32_t grid_x, uint32_t grid_y,
                     Timer tm) {
    // row classes per kind (xcd_tile): Q/K/V 2 (4 MB of activations, 5.6 MB of weights),
    // O 4 (8 MB, 4.5 MB), experts 8 (an expert tile's activations in one L2; its weights
    // are read by that tile only)
    PfGemm g = g0;
    g.xcd_rows = kind == QXP_QKV || kind == QXP_V_Q5 ? 2u : kind == QXP_O || kind == QXP_O_Q5 ? 4u : 8u;
    const uint32_t b = 8u / g.xcd_rows;
    if (grid_x % b) g.xcd_rows = 8u;   // (the column counts here are multiples of 8 workgroups)
    grid_y = (grid_y + g.xcd_rows - 1) / g.xcd_rows * g.xcd_rows;
    const dim3 grid(grid_x, grid_y);
    switch (kind) {
    case QXP_QKV:       // Q/K/V (or Q/K): IQ4_XS, 32 columns per wave
    case QXP_DOWN_IQ4:  // expert down, IQ4_XS (the kernel reads the expert groups from g)
        qx_launch(qxp_gemm<FMT_IQ4, 1, 1, EPI_STORE>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_O:         // O projection + residual: IQ4_XS
        qx_launch(qxp_gemm<FMT_IQ4, 1, 1, EPI_RESID>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_GU:        // expert gate/up + SwiGLU: IQ2_XS
        qx_launch(qxp_gemm<FMT_IQ2, 2, QXG_PF_EXPERT_MT, EPI_SWIGLU>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_DOWN:      // expert down: IQ3_XXS
        qx_launch(qxp_gemm<FMT_IQ3, 1, QXG_PF_EXPERT_MT, EPI_STORE>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_V_Q5:      // V alone: Q5_K
        qx_launch(qxp_gemm<FMT_Q5, 1, 1, EPI_STORE>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_O_Q5:      // O projection + residual: Q5_K
        qx_launch(qxp_gemm<FMT_Q5, 1, 1, EPI_RESID>, grid, dim3(256), 0, s, tm, g, P);
        break;
    case QXP_GU_IQ2S:   // expert gate/up + SwiGLU: IQ2_S
        qx_launch(qxp_gemm<FMT_IQ2S, 2, QXG_PF_EXPERT_MT, EPI_SWIGLU>, grid, dim3(256), 0, s, tm, g, P);
        break;
    default:            // expert down: IQ3_S
        qx_launch(qxp_gemm<FMT_IQ3S, 1, QXG_PF_EXPERT_MT, EPI_STORE>, grid, dim3(256), 0, s, tm, g, P);
        break;
    }
}
void qxp_launch_pack(hipStream_t s, int K, const float *src, const int32_t *map, const uint32_t *nrows, uint32_t rows,
                     uint32_t nvalid, uint4 *apk, float *rscale) {
    const dim3 grid((rows + 3) / 4);   // wave per row
    switch (K) {
    case 2048: hipLaunchKernelGGL(qxp_pack<2048>, grid, dim3(256), 0, s, src, map, nrows, rows, nvalid, apk, rscale); break;
    case 4096: hipLaunchKernelGGL(qxp_pack<4096>, grid, dim3(256), 0, s, src, map, nrows, rows, nvalid, apk, rscale); break;
    default: hipLaunchKernelGGL(qxp_pack<768>, grid, dim3(256), 0, s, src, map, nrows, rows, nvalid, apk, rscale); break;
    }
}
}
