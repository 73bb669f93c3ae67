// QXKVSNP1 KV snapshots: the reference's accumulated-KV file format
// (qx_write_accumulated_kv_snapshot / qx_read_accumulated_kv_snapshot,
// src/qx_format.c:5860-5968 of the reference), written from and read into the device
// INT8 cache.  Layout (little-endian):
//   header 48 B: "QXKVSNP1", version 2, layers, positions, ctx_tokens, kv_heads,
//                head_dim, format id (1 = int8), bytes per K or V row, next token, seed
//   per layer, per position < positions: K row, V row, K scale bits, V scale bits
//   SHA-256 (FIPS 180-4) of every preceding byte.
// Host code only; the device side is two copies per layer (qxg_kv_read / qxg_kv_write).
#include "qxg.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

// ---- SHA-256 (FIPS 180-4).  The round constants are the first 32 fraction bits of the
// cube roots of the first 64 primes and the initial state those of the square roots of
// the first 8 primes; both are derived here rather than tabulated.
struct Sha256Consts {
    uint32_t k[64], h0[8];
    Sha256Consts() {
        int primes[64], n = 0;
        for (int c = 2; n < 64; ++c) {
            bool p = true;
            for (int d = 2; d * d <= c; ++d) if (c % d == 0) { p = false; break; }
            if (p) primes[n++] = c;
        }
        for (int i = 0; i < 64; ++i) {
            const long double r = cbrtl((long double)primes[i]);
            k[i] = (uint32_t)((r - floorl(r)) * 4294967296.0L);
        }
        for (int i = 0; i < 8; ++i) {
            const long double r = sqrtl((long double)primes[i]);
            h0[i] = (uint32_t)((r - floorl(r)) * 4294967296.0L);
        }
    }
};
const Sha256Consts &sha_consts() {
    static const Sha256Consts c;
    return c;
}

inline uint32_t ror(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

struct Sha256 {
    uint32_t h[8];
    uint8_t buf[64];
    uint64_t total = 0;
    uint32_t fill = 0;
    Sha256() { memcpy(h, sha_consts().h0, sizeof(h)); }
    void block(const uint8_t *p) {
        const uint32_t *K = sha_consts().k;
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = ror(w[i - 15], 7) ^ ror(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = ror(w[i - 2], 17) ^ ror(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = hh + (ror(e, 6) ^ ror(e, 11) ^ ror(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
            const uint32_t t2 = (ror(a, 2) ^ ror(a, 13) ^ ror(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void update(const void *data, uint64_t n) {
        const uint8_t *p = static_cast<const uint8_t *>(data);
        total += n;
        while (n) {
            const uint32_t take = (uint32_t)(n < 64u - fill ? n : 64u - fill);
            memcpy(buf + fill, p, take);
            fill += take; p += take; n -= take;
            if (fill == 64) { block(buf); fill = 0; }
        }
    }
    void final(uint8_t out[32]) {
        const uint64_t bits = total * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

constexpr uint32_t SNAP_VERSION = 2, KV_HEADS = 4, HEAD_DIM = 128, FORMAT_INT8 = 1, ROW = 512;

void put32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
uint32_t get32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
void say(char *err, uint64_t n, const char *m) { if (err && n) snprintf(err, (size_t)n, "%s", m); }

// One layer's rows [0, positions) and scales as the file stores them.
struct LayerRows {
    std::vector<int8_t> k, v;
    std::vector<float> ks, vs;
    void size(uint32_t positions) { k.resize((size_t)positions * ROW); v.resize(k.size()); ks.resize(positions); vs.resize(positions); }
};

// Writer over a source that yields one layer at a time.
template <typename Src>
int write_snapshot(const char *path, uint32_t layers, uint32_t positions, uint32_t ctx_tokens, uint32_t next_token,
                   uint32_t seed, Src src, char *err, uint64_t n) {
    if (!path || !*path || !layers || !positions || positions > ctx_tokens) { say(err, n, "invalid accumulated KV snapshot output"); return 0; }
    FILE *fp = fopen(path, "wb");
    if (!fp) { say(err, n, "cannot open accumulated KV snapshot output"); return 0; }
    uint8_t hdr[48] = {0};
    memcpy(hdr, "QXKVSNP1", 8);
    const uint32_t f[10] = {SNAP_VERSION, layers, positions, ctx_tokens, KV_HEADS, HEAD_DIM, FORMAT_INT8, ROW, next_token, seed};
    for (int i = 0; i < 10; ++i) put32(hdr + 8 + 4 * i, f[i]);
    Sha256 sha;
    sha.update(hdr, sizeof(hdr));
    bool ok = fwrite(hdr, 1, sizeof(hdr), fp) == sizeof(hdr);
    LayerRows L;
    L.size(positions);
    for (uint32_t l = 0; l < layers && ok; ++l) {
        if (!src(l, L)) { fclose(fp); say(err, n, "cannot read the KV cache for the snapshot"); return 0; }
        for (uint32_t p = 0; p < positions && ok; ++p) {
            uint8_t sc[8];
            uint32_t bk, bv;
            memcpy(&bk, &L.ks[p], 4);
            memcpy(&bv, &L.vs[p], 4);
            put32(sc, bk);
            put32(sc + 4, bv);
            sha.update(&L.k[(size_t)p * ROW], ROW);
            sha.update(&L.v[(size_t)p * ROW], ROW);
            sha.update(sc, 8);
            ok = fwrite(&L.k[(size_t)p * ROW], 1, ROW, fp) == ROW && fwrite(&L.v[(size_t)p * ROW], 1, ROW, fp) == ROW &&
                 fwrite(sc, 1, 8, fp) == 8;
        }
    }
    uint8_t dig[32];
    sha.final(dig);
    if (ok) ok = fwrite(dig, 1, 32, fp) == 32;
    if (fclose(fp) != 0) ok = false;
    if (!ok) { say(err, n, "cannot write complete accumulated KV snapshot"); return 0; }
    return 1;
}

// Reader into a sink that takes one layer at a time (after the whole file verified).
template <typename Sink>
int read_snapshot(const char *path, uint32_t layers, uint32_t ctx_tokens, uint32_t seed, Sink sink,
                  uint32_t *positions_out, uint32_t *next_token_out, char *err, uint64_t n) {
    FILE *fp = path ? fopen(path, "rb") : nullptr;
    if (!fp) { say(err, n, "cannot open accumulated KV snapshot input"); return 0; }
    uint8_t hdr[48];
    bool ok = fread(hdr, 1, sizeof(hdr), fp) == sizeof(hdr);
    const uint32_t positions = ok ? get32(hdr + 16) : 0;
    if (!ok || memcmp(hdr, "QXKVSNP1", 8) != 0 || get32(hdr + 8) != SNAP_VERSION || get32(hdr + 12) != layers ||
        positions == 0 || positions > ctx_tokens || get32(hdr + 20) != ctx_tokens || get32(hdr + 24) != KV_HEADS ||
        get32(hdr + 28) != HEAD_DIM || get32(hdr + 32) != FORMAT_INT8 || get32(hdr + 36) != ROW || get32(hdr + 44) != seed) {
        fclose(fp);
        say(err, n, "accumulated KV snapshot header mismatch");
        return 0;
    }
    Sha256 sha;
    sha.update(hdr, sizeof(hdr));
    std::vector<LayerRows> all(layers);
    for (uint32_t l = 0; l < layers && ok; ++l) {
        LayerRows &L = all[l];
        L.size(positions);
        for (uint32_t p = 0; p < positions && ok; ++p) {
            uint8_t sc[8];
            ok = fread(&L.k[(size_t)p * ROW], 1, ROW, fp) == ROW && fread(&L.v[(size_t)p * ROW], 1, ROW, fp) == ROW &&
                 fread(sc, 1, 8, fp) == 8;
            if (!ok) break;
            sha.update(&L.k[(size_t)p * ROW], ROW);
            sha.update(&L.v[(size_t)p * ROW], ROW);
            sha.update(sc, 8);
            const uint32_t bk = get32(sc), bv = get32(sc + 4);
            memcpy(&L.ks[p], &bk, 4);
            memcpy(&L.vs[p], &bv, 4);
            if (!std::isfinite(L.ks[p]) || !std::isfinite(L.vs[p])) ok = false;
        }
    }
    uint8_t want[32], got[32];
    if (ok) ok = fread(want, 1, 32, fp) == 32;
    if (ok) {
        sha.final(got);
        ok = memcmp(want, got, 32) == 0;
    }
    if (ok && fgetc(fp) != EOF) ok = false;
    if (fclose(fp) != 0) ok = false;
    if (!ok) { say(err, n, "accumulated KV snapshot payload mismatch"); return 0; }
    for (uint32_t l = 0; l < layers; ++l)
        if (!sink(l, all[l], positions)) { say(err, n, "cannot write the KV cache from the snapshot"); return 0; }
    if (positions_out) *positions_out = positions;
    if (next_token_out) *next_token_out = get32(hdr + 40);
    return 1;
}
}  // namespace

extern "C" {

int qxg_kvsnap_write(const char *path, uint32_t layers, uint32_t positions, uint32_t ctx_tokens, uint32_t next_token,
                     uint32_t seed, const int8_t *k, const int8_t *v, const float *kscale, const float *vscale,
                     char *err, uint64_t err_len) {
    if (!k || !v || !kscale || !vscale) { say(err, err_len, "invalid accumulated KV snapshot output"); return 0; }
    return write_snapshot(path, layers, positions, ctx_tokens, next_token, seed, [&](uint32_t l, LayerRows &L) {
        const size_t slot = (size_t)l * ctx_tokens;
        memcpy(L.k.data(), k + slot * ROW, L.k.size());
        memcpy(L.v.data(), v + slot * ROW, L.v.size());
        memcpy(L.ks.data(), kscale + slot, L.ks.size() * 4);
        memcpy(L.vs.data(), vscale + slot, L.vs.size() * 4);
        return true;
    }, err, err_len);
}

int qxg_kvsnap_read(const char *path, uint32_t layers, uint32_t ctx_tokens, uint32_t seed, int8_t *k, int8_t *v,
                    float *kscale, float *vscale, uint32_t *positions_out, uint32_t *next_token_out, char *err,
                    uint64_t err_len) {
    if (!k || !v || !kscale || !vscale) { say(err, err_len, "invalid accumulated KV snapshot input"); return 0; }
    return read_snapshot(path, layers, ctx_tokens, seed, [&](uint32_t l, const LayerRows &L, uint32_t positions) {
        const size_t slot = (size_t)l * ctx_tokens;
        memcpy(k + slot * ROW, L.k.data(), (size_t)positions * ROW);
        memcpy(v + slot * ROW, L.v.data(), (size_t)positions * ROW);
        memcpy(kscale + slot, L.ks.data(), (size_t)positions * 4);
        memcpy(vscale + slot, L.vs.data(), (size_t)positions * 4);
        return true;
    }, positions_out, next_token_out, err, err_len);
}

int qxg_kv_export(qxg_ctx *ctx, const char *path, uint32_t layers, uint32_t positions, uint32_t ctx_tokens,
                  uint32_t next_token, uint32_t seed, char *err, uint64_t err_len) {
    if (!ctx) { say(err, err_len, "invalid context"); return 0; }
    return write_snapshot(path, layers, positions, ctx_tokens, next_token, seed, [&](uint32_t l, LayerRows &L) {
        return qxg_kv_read(ctx, l, 0, positions, L.k.data(), L.v.data(), L.ks.data(), L.vs.data(), err, err_len) == 1;
    }, err, err_len);
}

int qxg_kv_import(qxg_ctx *ctx, const char *path, uint32_t layers, uint32_t ctx_tokens, uint32_t seed,
                  uint32_t *positions_out, uint32_t *next_token_out, char *err, uint64_t err_len) {
    if (!ctx) { say(err, err_len, "invalid context"); return 0; }
    return read_snapshot(path, layers, ctx_tokens, seed, [&](uint32_t l, const LayerRows &L, uint32_t positions) {
        return qxg_kv_write(ctx, l, 0, positions, L.k.data(), L.v.data(), L.ks.data(), L.vs.data(), err, err_len) == 1;
    }, positions_out, next_token_out, err, err_len);
}

}  // extern "C"
