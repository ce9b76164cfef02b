/* fronk_oracle.c - CPU restatement of the reference expert-slice path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Nothing in fronk_amd/ or include/
 * links or calls it. Each function names the reference lines it follows; the
 * arithmetic, loop order and double accumulation are kept exactly because the
 * golden corpus and the parity tests depend on them.
 */
#include "fronk_oracle.h"
#include <fenv.h>
#include <float.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

/* ---------------------------------------------------------------- scalars */

/* IEEE binary16 -> binary32, exact, subnormals via ldexpf (src/q4.c:12-20). */
float fo_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) {
        float f = ldexpf((float)m, -24);
        return sign ? -f : f;
    }
    uint32_t bits = sign | (e == 31 ? 0x7f800000u : (e + 112u) << 23) | m << 13;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (uint16_t)p[1] << 8); }

/* Bytes per row of n weights (src/native.h:19-21, src/model.h:21-23). */
uint64_t fo_row_bytes(unsigned type, unsigned n) {
    switch (type) {
    case FO_Q4_K: return (uint64_t)n / 256 * 144;
    case FO_MXFP4: return (uint64_t)n / 32 * 17;
    case FO_Q8_0: return (uint64_t)n / 32 * 34;
    case FO_Q4_0: return (uint64_t)n / 32 * 18;
    default: return 0;
    }
}

/* Layout of a 48-layer unit: per layer, 512 routed slices then the shared
 * slice; per slice, 32 gate rows, 32 up rows, then the down matrix
 * (src/native.h:9-18; legacy src/backend.h:37-50). */
int fo_layout_get(unsigned hidden, unsigned format, fo_layout *out) {
    if (!out || !hidden || hidden > FO_MAX_HIDDEN || hidden % 32) return FO_INVALID;
    fo_layout l;
    memset(&l, 0, sizeof(l));
    l.hidden = hidden;
    l.format = format;
    switch (format) {
    case FO_FMT_LEGACY: l.gu_type = l.down_type = FO_Q4_0; break;
    case FO_FMT_NATIVE: l.gu_type = FO_Q4_K; l.down_type = FO_MXFP4; break;
    case FO_FMT_Q4KT: l.gu_type = l.down_type = FO_Q4_K; l.down_transposed = 1; break;
    case FO_FMT_Q8: l.gu_type = l.down_type = FO_Q8_0; break;
    case FO_FMT_MXFP4: l.gu_type = l.down_type = FO_MXFP4; break;
    default: return FO_INVALID;
    }
    if ((l.gu_type == FO_Q4_K || l.down_transposed) && hidden % 256) return FO_INVALID;
    l.gu_row = fo_row_bytes(l.gu_type, hidden);
    l.proj = FO_NEURONS * l.gu_row;
    l.down_row = l.down_transposed ? fo_row_bytes(l.down_type, hidden) : fo_row_bytes(l.down_type, FO_NEURONS);
    l.down = l.down_transposed ? FO_NEURONS * l.down_row : (uint64_t)hidden * l.down_row;
    l.slice = 2 * l.proj + l.down;
    if (format == FO_FMT_LEGACY) {
        l.shared_gu_type = l.shared_down_type = FO_Q4_0;
        l.shared_proj = l.proj;
        l.shared_down = l.down;
        l.shared_slice = l.slice;
    } else {
        l.shared_gu_type = l.shared_down_type = FO_Q8_0;
        l.shared_proj = (uint64_t)hidden / 32 * 34 * FO_NEURONS;
        l.shared_down = (uint64_t)hidden * 34;
        l.shared_slice = 3 * l.shared_proj;
    }
    l.layer = FO_ROUTED * l.slice + l.shared_slice;
    l.block = FO_LAYERS * l.layer;
    *out = l;
    return FO_OK;
}

/* fr_native_offset / fr_slice_offset (src/native.h:16-18, src/backend.h:48-50). */
uint64_t fo_slice_offset(const fo_layout *l, unsigned layer, unsigned expert) {
    return (uint64_t)layer * l->layer + (uint64_t)expert * l->slice;
}

/* Legacy canonical Q4_0 dot in double (src/q4.c:22-35): 18-byte groups, byte
 * j's low nibble is weight j, high nibble weight j+16, w = (q-8)*d. */
int fo_q4_dot(const uint8_t *q, const float *x, size_t n, double *out) {
    if (!q || !x || !out || !n || n % 32) return FO_INVALID;
    double sum = 0;
    for (size_t k = 0; k < n; k += 32, q += 18) {
        float d = fo_f16(le16(q));
        if (!isfinite(d)) return FO_NUMERIC;
        for (unsigned j = 0; j < 32; ++j) {
            int v = (j < 16 ? q[2 + j] & 15 : q[2 + j - 16] >> 4) - 8;
            sum += ((double)v * d) * x[k + j];
        }
    }
    if (!isfinite(sum)) return FO_NUMERIC;
    *out = sum;
    return FO_OK;
}

/* ref-q8 activation quantizer (src/q4.c:37-61): groups of 64 (the last may be
 * 32), fp32 scale max/127, fp32 multiplier 127/max (or (v/max)*127 when the
 * multiplier overflows), nearest-even, clamp +-127, dequantize through double
 * and cap at +-FLT_MAX. Zero groups and underflowing scales give zeros. */
int fo_q8_activation(const float *x, float *out, size_t n) {
    if (!x || !out || !n || n % 32 || fegetround() != FE_TONEAREST) return FO_INVALID;
    for (size_t k = 0; k < n; k += 64) {
        size_t count = n - k < 64 ? n - k : 64;
        float max = 0;
        for (size_t j = 0; j < count; ++j) {
            if (!isfinite(x[k + j])) return FO_NUMERIC;
            if (fabsf(x[k + j]) > max) max = fabsf(x[k + j]);
        }
        float scale = max / 127.0f;
        if (scale == 0) {
            for (size_t j = 0; j < count; ++j) out[k + j] = 0;
            continue;
        }
        float inv = 127.0f / max;
        for (size_t j = 0; j < count; ++j) {
            float v = isfinite(inv) ? x[k + j] * inv : (x[k + j] / max) * 127.0f;
            v = nearbyintf(v);
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            double back = (double)v * scale;
            if (back > FLT_MAX) back = FLT_MAX;
            if (back < -FLT_MAX) back = -FLT_MAX;
            out[k + j] = (float)back;
        }
    }
    return FO_OK;
}

/* cvtps2dq: nearest-even, NaN or out of range -> INT32_MIN. */
static int32_t cvt_ps_epi32(float v) {
    if (isnan(v) || v >= 2147483648.0f || v < -2147483648.0f) return INT32_MIN;
    return (int32_t)nearbyintf(v);
}
static int32_t sat(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : v > hi ? hi : v; }

/* AVX2 backend activation quantizer (backends/avx2.c:184-203): per group of
 * `group` values, amax, d = amax/127, inv = amax ? 127/amax : 0 (no overflow
 * fallback), cvtps rounding, saturating int32->int16->int8 packs, and an int16
 * sum of the unsaturated int32 codes per 32 values (wrapping arithmetic). */
void fo_quantize8(const float *x, unsigned n, unsigned group, int8_t *q, float *d, int16_t *s) {
    for (unsigned i = 0; i < n; i += group) {
        float amax = 0;
        for (unsigned j = 0; j < group; ++j) {
            float a = fabsf(x[i + j]);
            if (a > amax) amax = a;
        }
        d[i / group] = amax / 127.0f;
        float inv = amax != 0 ? 127.0f / amax : 0;
        for (unsigned j = 0; j < group; j += 32) {
            uint32_t sum = 0;
            for (unsigned k = 0; k < 32; ++k) {
                int32_t v = cvt_ps_epi32(x[i + j + k] * inv);
                sum += (uint32_t)v;
                q[i + j + k] = (int8_t)sat(sat(v, -32768, 32767), -128, 127);
            }
            if (s) s[(i + j) / 32] = (int16_t)(uint16_t)sum;
        }
    }
}

static const float mx_lut[16] = {0, .5f, 1, 1.5f, 2, 3, 4, 6, 0, -.5f, -1, -1.5f, -2, -3, -4, -6};

/* Q4_K sub-block scale and min for group g of a 144-byte super-block:
 * 6-bit values, groups 4..7 split over three bytes (src/native.c:14-19). */
static void q4k_scale_min(const uint8_t *s, unsigned g, unsigned *sc, unsigned *mi) {
    if (g < 4) {
        *sc = s[g] & 63;
        *mi = s[g + 4] & 63;
    } else {
        *sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
        *mi = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

/* One weight of a row, exactly as fr_native_dot decodes it
 * (src/native.c:13-31): Q4_K w = (d*sc)*q - dmin*mi; MXFP4 w = 2^(e-127) *
 * E2M1(code); Q8_0 w = d*int8; Q4_0 w = (q-8)*d (src/q4.c:29-31). */
float fo_decode(const uint8_t *p, unsigned type, unsigned j) {
    if (type == FO_Q4_K) {
        const uint8_t *b = p + (size_t)(j / 256) * 144;
        unsigned g = j % 256 / 32, sc, mi;
        q4k_scale_min(b + 4, g, &sc, &mi);
        float d = fo_f16(le16(b)), m = fo_f16(le16(b + 2));
        unsigned q = (b[16 + (g / 2) * 32 + j % 32] >> ((g % 2) * 4)) & 15;
        return (d * (float)sc) * (float)q - m * (float)mi;
    }
    if (type == FO_MXFP4) {
        const uint8_t *b = p + (size_t)(j / 32) * 17;
        if (b[0] == 255) return NAN;
        return ldexpf(1.0f, (int)b[0] - 127) * mx_lut[(b[1 + j % 16] >> ((j % 32 / 16) * 4)) & 15];
    }
    if (type == FO_Q8_0) {
        const uint8_t *b = p + (size_t)(j / 32) * 34;
        return fo_f16(le16(b)) * (float)(int8_t)b[2 + j % 32];
    }
    if (type == FO_Q4_0) {
        const uint8_t *b = p + (size_t)(j / 32) * 18;
        unsigned k = j % 32;
        int v = (k < 16 ? b[2 + k] & 15 : b[2 + k - 16] >> 4) - 8;
        return (float)v * fo_f16(le16(b));
    }
    return NAN;
}

int fo_dequant_row(const uint8_t *row, unsigned type, unsigned n, float *out) {
    if (!row || !out || !n) return FO_INVALID;
    for (unsigned j = 0; j < n; ++j) out[j] = fo_decode(row, type, j);
    return FO_OK;
}

/* fr_native_dot (src/native.c:7-37): double sum in column order; a non-finite
 * weight, input or sum is FO_NUMERIC; a partial block is FO_INVALID. */
int fo_native_dot(const uint8_t *p, unsigned type, const float *x, unsigned n, double *out) {
    if (!p || !x || !out || !n || (type != FO_Q4_K && type != FO_MXFP4 && type != FO_Q8_0) ||
        n % (type == FO_Q4_K ? 256 : 32))
        return FO_INVALID;
    double sum = 0;
    for (unsigned j = 0; j < n; ++j) {
        float w = fo_decode(p, type, j);
        if (!isfinite(w) || !isfinite(x[j])) return FO_NUMERIC;
        sum += (double)w * x[j];
    }
    if (!isfinite(sum)) return FO_NUMERIC;
    *out = sum;
    return FO_OK;
}

/* ------------------------------------------------------------- ref run() */

static int narrow(double v, float *out) {
    if (!isfinite(v) || fabs(v) > FLT_MAX) return FO_NUMERIC;
    *out = (float)v;
    return FO_OK;
}

/* Request validation in the reference order (backends/ref.c:41-56). */
static int validate(const fo_req *r) {
    if (!r || r->layer >= FO_LAYERS || r->burst < 1 || r->burst > FO_MAX_BURST ||
        fegetround() != FE_TONEAREST)
        return FO_INVALID;
    for (unsigned t = 0; t < r->burst; ++t) {
        for (unsigned e = 0; e < FO_ACTIVE_ROUTED; ++e) {
            if (r->expert[t][e] >= FO_ROUTED) return FO_INVALID;
            for (unsigned j = 0; j < e; ++j)
                if (r->expert[t][j] == r->expert[t][e]) return FO_INVALID;
        }
        for (unsigned e = 0; e < FO_ACTIVE; ++e) {
            if (!isfinite(r->gate[t][e])) return FO_NUMERIC;
            if (r->gate[t][e] < 0) return FO_INVALID;
        }
        for (unsigned d = 0; d < r->hidden; ++d)
            if (!isfinite(r->x[t][d])) return FO_NUMERIC;
    }
    return FO_OK;
}

static int row_dot(const uint8_t *row, unsigned type, const float *x, unsigned n, double *out) {
    return type == FO_Q4_0 ? fo_q4_dot(row, x, n, out) : fo_native_dot(row, type, x, n, out);
}

/* Down contribution of one slice to y (backends/ref.c:86-92). The stored
 * [H x 32] orientation dots row d with h; the transposed [32 x H] orientation
 * reads element (n, d) of row n, still summing n = 0..31 in double. */
static int down_add(const uint8_t *down, const fo_layout *l, unsigned type, int transposed,
                    const float *h, double gate, double *y) {
    unsigned H = l->hidden;
    for (unsigned d = 0; d < H; ++d) {
        double dot = 0;
        if (!transposed) {
            int rc = row_dot(down + (size_t)d * fo_row_bytes(type, FO_NEURONS), type, h, FO_NEURONS, &dot);
            if (rc) return rc;
        } else {
            uint64_t rowb = fo_row_bytes(type, H);
            for (unsigned n = 0; n < FO_NEURONS; ++n) {
                float w = fo_decode(down + n * rowb, type, d);
                if (!isfinite(w) || !isfinite(h[n])) return FO_NUMERIC;
                dot += (double)w * h[n];
            }
            if (!isfinite(dot)) return FO_NUMERIC;
        }
        y[d] += gate * dot;
    }
    return FO_OK;
}

/* ref / ref-q8 run (backends/ref.c:57-98): token-first; routed experts in
 * request order, then the shared expert unless its gate is 0; ascending
 * loaded block; gate/up dots narrowed to float; h = float(a*sigmoid(a)*u) in
 * double with the stable sigmoid; y accumulated in double and narrowed once.
 * ref-q8 quantizes x (groups of 64) and each slice's h (one group of 32). */
int fo_ref_run(const uint8_t *const blocks[FO_BLOCKS], unsigned format, int q8,
               const fo_req *req, float *y_out) {
    if (!y_out || !blocks) return FO_INVALID;
    int rc = validate(req);
    if (rc) return rc;
    fo_layout l;
    if (fo_layout_get(req->hidden, format, &l)) return FO_INVALID;
    int any = 0;
    for (int b = 0; b < FO_BLOCKS; ++b) any |= blocks[b] != NULL;
    if (!any) return FO_STATE;
    unsigned H = req->hidden;
    static double y[FO_MAX_HIDDEN];
    static float quantized[FO_MAX_HIDDEN];
    static float result[FO_MAX_BURST][FO_MAX_HIDDEN];
    for (unsigned t = 0; t < req->burst; ++t) {
        memset(y, 0, sizeof(y));
        const float *x = req->x[t];
        if (q8) {
            rc = fo_q8_activation(x, quantized, H);
            if (rc) return rc;
            x = quantized;
        }
        for (unsigned e = 0; e < FO_ACTIVE; ++e) {
            int shared = e == FO_ACTIVE_ROUTED;
            if (shared && req->gate[t][e] == 0) continue;
            unsigned id = shared ? FO_SHARED : req->expert[t][e];
            unsigned gu = shared ? l.shared_gu_type : l.gu_type;
            unsigned dn = shared ? l.shared_down_type : l.down_type;
            int transposed = shared ? 0 : (int)l.down_transposed;
            uint64_t proj = shared ? l.shared_proj : l.proj, gu_row = fo_row_bytes(gu, H);
            for (unsigned b = 0; b < FO_BLOCKS; ++b) {
                if (!blocks[b]) continue;
                const uint8_t *p = blocks[b] + fo_slice_offset(&l, req->layer, id);
                float h[FO_NEURONS];
                for (unsigned n = 0; n < FO_NEURONS; ++n) {
                    double ad, ud;
                    float a, u;
                    rc = row_dot(p + n * gu_row, gu, x, H, &ad);
                    if (rc) return rc;
                    rc = row_dot(p + proj + n * gu_row, gu, x, H, &ud);
                    if (rc) return rc;
                    if (narrow(ad, &a) || narrow(ud, &u)) return FO_NUMERIC;
                    double sigmoid = a >= 0 ? 1 / (1 + exp(-(double)a)) : exp((double)a) / (1 + exp((double)a));
                    if (narrow((double)a * sigmoid * u, &h[n])) return FO_NUMERIC;
                }
                if (q8) {
                    rc = fo_q8_activation(h, h, FO_NEURONS);
                    if (rc) return rc;
                }
                rc = down_add(p + 2 * proj, &l, dn, transposed, h, (double)req->gate[t][e], y);
                if (rc) return rc;
            }
        }
        for (unsigned d = 0; d < H; ++d)
            if (narrow(y[d], &result[t][d])) return FO_NUMERIC;
    }
    for (unsigned t = 0; t < req->burst; ++t) memcpy(y_out + (size_t)t * H, result[t], H * sizeof(float));
    return FO_OK;
}

/* ---------------------------------------------------------------- metrics */

/* fr_compare (src/backend.c:74-92): per-token relative L2, normalized max and
 * cosine in double; a zero reference needs an exactly zero candidate. */
int fo_compare(const float *ref, const float *act, size_t n, double out[3]) {
    if (!ref || !act || !out || !n) return FO_INVALID;
    double r2 = 0, a2 = 0, d2 = 0, dot = 0, rmax = 0, dmax = 0;
    for (size_t i = 0; i < n; ++i) {
        double r = ref[i], a = act[i], d = a - r;
        if (!isfinite(r) || !isfinite(a)) return FO_NUMERIC;
        r2 += r * r;
        a2 += a * a;
        d2 += d * d;
        dot += r * a;
        if (fabs(r) > rmax) rmax = fabs(r);
        if (fabs(d) > dmax) dmax = fabs(d);
    }
    if (r2 == 0) {
        out[0] = a2 != 0 ? INFINITY : 0;
        out[1] = a2 != 0 ? INFINITY : 0;
        out[2] = a2 != 0 ? 0 : 1;
    } else {
        out[0] = sqrt(d2 / r2);
        out[1] = dmax / rmax;
        out[2] = a2 != 0 ? dot / (sqrt(r2) * sqrt(a2)) : 0;
        if (out[2] > 1) out[2] = 1;
        if (out[2] < -1) out[2] = -1;
    }
    return FO_OK;
}

/* fr_conforms (src/backend.c:93-97): inclusive limits, finite metrics. */
int fo_conforms(const double e[3], const double t[3]) {
    return e && t && isfinite(e[0]) && isfinite(e[1]) && isfinite(e[2]) && e[0] >= 0 && e[1] >= 0 &&
           e[2] >= -1 && e[2] <= 1 && e[0] <= t[0] && e[1] <= t[1] && e[2] >= t[2];
}

/* ---------------------------------------------------------------- SHA-256 */

/* FIPS 180-4 SHA-256 (the reference digests fixtures with its own
 * src/sha256.c; any conforming implementation gives the same bytes). */
typedef struct { uint32_t h[8]; uint64_t bits; uint8_t buf[64]; unsigned used; } sha_ctx;
static const uint32_t sha_k[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
static uint32_t rotr(uint32_t x, unsigned n) { return x >> n | x << (32 - n); }
static void sha_block(sha_ctx *c, const uint8_t *p) {
    uint32_t w[64];
    for (unsigned i = 0; i < 16; ++i)
        w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (unsigned i = 16; i < 64; ++i) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = c->h[0], b = c->h[1], cc = c->h[2], d = c->h[3], e = c->h[4], f = c->h[5], g = c->h[6], h = c->h[7];
    for (unsigned i = 0; i < 64; ++i) {
        uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + sha_k[i] + w[i];
        uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & cc) ^ (b & cc));
        h = g; g = f; f = e; e = d + t1; d = cc; cc = b; b = a; a = t1 + t2;
    }
    c->h[0] += a; c->h[1] += b; c->h[2] += cc; c->h[3] += d;
    c->h[4] += e; c->h[5] += f; c->h[6] += g; c->h[7] += h;
}
static void sha_init(sha_ctx *c) {
    static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->h, iv, sizeof(iv));
    c->bits = 0;
    c->used = 0;
}
static void sha_update(sha_ctx *c, const void *data, size_t len) {
    const uint8_t *p = data;
    c->bits += (uint64_t)len * 8;
    while (len) {
        size_t take = 64 - c->used < len ? 64 - c->used : len;
        memcpy(c->buf + c->used, p, take);
        c->used += (unsigned)take;
        p += take;
        len -= take;
        if (c->used == 64) {
            sha_block(c, c->buf);
            c->used = 0;
        }
    }
}
static void sha_final(sha_ctx *c, uint8_t out[32]) {
    uint64_t bits = c->bits;
    uint8_t pad = 0x80, zero = 0, len[8];
    sha_update(c, &pad, 1);
    while (c->used != 56) sha_update(c, &zero, 1);
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    sha_update(c, len, 8);
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)(c->h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(c->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->h[i] >> 8);
        out[4 * i + 3] = (uint8_t)c->h[i];
    }
}
void fo_sha256(const void *data, size_t len, uint8_t out[32]) {
    sha_ctx c;
    sha_init(&c);
    sha_update(&c, data, len);
    sha_final(&c, out);
}
static void sha_u32(sha_ctx *c, uint32_t v) {
    uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    sha_update(c, b, 4);
}
static void sha_f32(sha_ctx *c, float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    sha_u32(c, bits);
}

/* --------------------------------------------------- golden corpus recipe */

/* Fixture table (src/vectors.c:12-17): name, burst, layer, owned-block mask. */
static const struct { const char *name; unsigned burst, layer; uint32_t mask; } vcases[8] = {
    {"zero-input", 1, 0, 1},       {"zero-gates", 2, 1, 1u << 19},
    {"signed", 1, 0, 1},           {"reused", 4, 17, 1u << 7},
    {"mixed", 8, 47, 1u | (1u << 19)}, {"outliers", 2, 31, 1u << 19},
    {"tiny", 1, 23, 1u << 11},     {"all-blocks", 1, 1, (1u << 20) - 1}};

/* xorshift32 with shifts 13, 17, 5 (src/vectors.c:19). */
static uint32_t xorshift32(uint32_t *s) {
    *s ^= *s << 13;
    *s ^= *s >> 17;
    *s ^= *s << 5;
    return *s;
}

/* Request of fixture `index` (src/vectors.c:36-53): routed ids, gates and
 * activations from the per-index seed 0x6d2b79f5+index; H = 2560. */
int fo_vector_request(unsigned index, fo_req *r, uint32_t *mask, char name[16]) {
    if (index >= 8 || !r) return FO_INVALID;
    memset(r, 0, sizeof(*r));
    r->hidden = 2560;
    r->layer = vcases[index].layer;
    r->burst = vcases[index].burst;
    if (mask) *mask = vcases[index].mask;
    if (name) snprintf(name, 16, "%s", vcases[index].name);
    uint32_t seed = 0x6d2b79f5u + index;
    for (unsigned t = 0; t < r->burst; ++t) {
        for (unsigned e = 0; e < FO_ACTIVE_ROUTED; ++e) {
            unsigned id = index == 4 ? t * 10 + e : e == 0 ? 0 : e == 1 ? 511 : e * 47 + 13;
            if (index == 4 && t == 7 && e == 9) id = 511;
            r->expert[t][e] = (uint16_t)id;
        }
        for (unsigned e = 0; e < FO_ACTIVE; ++e)
            r->gate[t][e] = index == 1 ? 0 : e == FO_ACTIVE_ROUTED ? 0.75f : (float)((e + t) % 5) * 0.03125f;
        for (unsigned d = 0; d < 2560; ++d) {
            float x = (float)((int)(xorshift32(&seed) % 8193) - 4096) * 0x1p-12f;
            if (index == 0) x = 0;
            if (index == 5) x = d % 127 == 0 ? (d % 2 ? 16.0f : -16.0f) : x * 0.015625f;
            if (index == 6) x *= 0x1p-12f;
            r->x[t][d] = x;
        }
    }
    return FO_OK;
}

/* Materialize the used legacy Q4_0 slices of every owned block and return the
 * SHA-256 digest binding request and weights (src/vectors.c:54-82). Each slice
 * is seeded from (block, expert, layer); scales are signed fp16 near 2^-7 (gate,
 * up) or 2^-6 (down) with every 257th group subnormal or zero. */
int fo_vector_fill(unsigned index, uint8_t *const blocks[FO_BLOCKS], char digest[65]) {
    fo_req r;
    uint32_t mask;
    if (fo_vector_request(index, &r, &mask, NULL)) return FO_INVALID;
    fo_layout l;
    fo_layout_get(2560, FO_FMT_LEGACY, &l);
    uint8_t used[FO_EXPERTS] = {0};
    used[FO_SHARED] = 1;
    for (unsigned t = 0; t < r.burst; ++t)
        for (unsigned e = 0; e < FO_ACTIVE_ROUTED; ++e) used[r.expert[t][e]] = 1;
    sha_ctx h;
    sha_init(&h);
    sha_u32(&h, index);
    sha_u32(&h, r.layer);
    sha_u32(&h, r.burst);
    sha_u32(&h, mask);
    for (unsigned t = 0; t < r.burst; ++t) {
        for (unsigned e = 0; e < FO_ACTIVE_ROUTED; ++e) sha_u32(&h, r.expert[t][e]);
        for (unsigned e = 0; e < FO_ACTIVE; ++e) sha_f32(&h, r.gate[t][e]);
        for (unsigned d = 0; d < 2560; ++d) sha_f32(&h, r.x[t][d]);
    }
    size_t groups = l.slice / 18, down_first = 2 * l.proj / 18;
    for (unsigned b = 0; b < FO_BLOCKS; ++b) {
        if (!(mask & (1u << b))) continue;
        if (!blocks || !blocks[b]) return FO_INVALID;
        for (unsigned e = 0; e < FO_EXPERTS; ++e) {
            if (!used[e]) continue;
            uint32_t seed = 0x9e3779b9u ^ (b * 0x85ebca6bu) ^ (e * 0xc2b2ae35u) ^ (r.layer * 0x27d4eb2du);
            uint8_t *slice = blocks[b] + fo_slice_offset(&l, r.layer, e);
            for (size_t k = 0; k < groups; ++k) {
                uint32_t bits = xorshift32(&seed);
                uint16_t scale = (uint16_t)((k >= down_first ? 0x2400 : 0x2000) | (bits & 1023));
                if (bits & 1024) scale |= 0x8000;
                if (k % 257 == 0) scale = (uint16_t)(bits & 0x83ff);
                uint8_t *q = slice + k * 18;
                q[0] = (uint8_t)scale;
                q[1] = (uint8_t)(scale >> 8);
                for (int j = 0; j < 16; ++j) q[2 + j] = (uint8_t)(xorshift32(&seed) >> 24);
            }
            sha_update(&h, slice, l.slice);
        }
    }
    uint8_t sum[32];
    sha_final(&h, sum);
    static const char hex[] = "0123456789abcdef";
    for (int i = 0; i < 32; ++i) {
        digest[2 * i] = hex[sum[i] >> 4];
        digest[2 * i + 1] = hex[sum[i] & 15];
    }
    digest[64] = 0;
    return FO_OK;
}

/* Golden file text (src/vectors.c:120-125): header line, then token-major
 * outputs as C99 hex floats, 16 per line. */
int fo_vector_format(unsigned index, const fo_req *r, uint32_t mask, const char *digest,
                     const float *y, char *out, size_t cap, size_t *len) {
    if (index >= 8 || !r || !digest || !y || !out || !len) return FO_INVALID;
    size_t used = 0;
    int n = snprintf(out, cap, "FRV1 %s %u %u %u %s\n", vcases[index].name, r->layer, r->burst, mask, digest);
    if (n < 0 || (size_t)n >= cap) return FO_INVALID;
    used = (size_t)n;
    for (unsigned t = 0; t < r->burst; ++t)
        for (unsigned d = 0; d < 2560; ++d) {
            n = snprintf(out + used, cap - used, "%a%c", (double)y[t * 2560 + d], d % 16 == 15 ? '\n' : ' ');
            if (n < 0 || (size_t)n >= cap - used) return FO_INVALID;
            used += (size_t)n;
        }
    *len = used;
    return FO_OK;
}

/* ------------------------------------------------ native fixture recipe */

/* LCG 1664525, 1013904223 (src/native.c:39). */
uint32_t fo_lcg(uint32_t *s) {
    *s = *s * 1664525u + 1013904223u;
    return *s;
}

/* One row of `n` weights of random bytes with fixed finite scales
 * (src/native.c:40-48): Q4_K d = 2^-13, dmin = 2^-10; Q8_0 d = 2^-8;
 * MXFP4 exponent 120..124. */
static void fixture_row(uint8_t *p, unsigned type, unsigned n, uint32_t *seed) {
    unsigned count = n / (type == FO_Q4_K ? 256 : 32);
    unsigned bytes = type == FO_Q4_K ? 144 : type == FO_Q8_0 ? 34 : 17;
    for (unsigned i = 0; i < count; ++i, p += bytes) {
        for (unsigned j = 0; j < bytes; ++j) p[j] = (uint8_t)(fo_lcg(seed) >> 24);
        if (type == FO_Q4_K) {
            p[0] = 0; p[1] = 0x08; p[2] = 0; p[3] = 0x14;
        } else if (type == FO_Q8_0) {
            p[0] = 0; p[1] = 0x1c;
        } else {
            p[0] = (uint8_t)(120 + fo_lcg(seed) % 5);
        }
    }
}

/* fill_slice (src/native.c:49-57): gate row n and up row n interleaved, then
 * every down row. The transposed down of Q4KT is 32 rows of H. */
void fo_fill_slice(uint8_t *p, const fo_layout *l, unsigned id, uint32_t *seed) {
    int shared = id == FO_SHARED;
    unsigned gu = shared ? l->shared_gu_type : l->gu_type, dn = shared ? l->shared_down_type : l->down_type;
    uint64_t proj = shared ? l->shared_proj : l->proj, row = fo_row_bytes(gu, l->hidden);
    for (unsigned n = 0; n < FO_NEURONS; ++n) {
        fixture_row(p + n * row, gu, l->hidden, seed);
        fixture_row(p + proj + n * row, gu, l->hidden, seed);
    }
    if (!shared && l->down_transposed) {
        uint64_t drow = fo_row_bytes(dn, l->hidden);
        for (unsigned n = 0; n < FO_NEURONS; ++n) fixture_row(p + 2 * proj + n * drow, dn, l->hidden, seed);
    } else {
        uint64_t drow = fo_row_bytes(dn, FO_NEURONS);
        for (unsigned d = 0; d < l->hidden; ++d) fixture_row(p + 2 * proj + d * drow, dn, FO_NEURONS, seed);
    }
}

/* ------------------------------------------------------------------------
 * Synthetic measurement weights (not a reference function). Distributions:
 * Q4_K nibbles and 6-bit scales/mins uniform, d and dmin = fp16(U[1e-3,1e-2]);
 * Q8_0 int8 uniform on [-127, 127] with an fp16(U[1e-3,1e-2]) scale; MXFP4
 * codes uniform over the 16 values with E8M0 uniform on [118, 130]; Q4_0
 * nibbles uniform with an fp16(U[1e-3,1e-2]) scale. Every byte is a pure
 * function of (seed, block, layer, expert, byte offset in the slice), so a
 * generator on the device can write the same bytes in any order or layout.
 * The hash is the splitmix64 finaliser (Steele, Lea, Flood 2014). */
static uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t fo_synth_key(uint64_t seed, unsigned block, unsigned layer, unsigned expert) {
    return mix64(seed) ^ ((uint64_t)block << 54) ^ ((uint64_t)layer << 44) ^ ((uint64_t)expert << 32);
}

static uint64_t synth_hash(uint64_t key, unsigned domain, uint64_t word) {
    return mix64(key ^ ((uint64_t)domain << 60) ^ word);
}

/* fp16 bits of 1e-3 + 9e-3*u, u = the top 24 bits of h over 2^24, rounded to
 * nearest even; the value is a normal binary16 (exponent field 5..8). */
uint16_t fo_synth_scale(uint64_t h) {
    double u = (double)(h >> 40) * 0x1p-24;
    double v = 1e-3 + 9e-3 * u;
    uint64_t bits;
    memcpy(&bits, &v, sizeof(bits));
    int e = (int)((bits >> 52) & 0x7ff) - 1023 + 15;
    uint64_t mant = bits & ((1ull << 52) - 1), q = mant >> 42, rem = mant & ((1ull << 42) - 1);
    if (rem > (1ull << 41) || (rem == (1ull << 41) && (q & 1))) ++q;
    if (q == 1024) {
        q = 0;
        ++e;
    }
    return (uint16_t)((unsigned)e << 10 | (unsigned)q);
}

static unsigned type_block_bytes(unsigned type) {
    return type == FO_Q4_K ? 144 : type == FO_Q8_0 ? 34 : type == FO_MXFP4 ? 17 : 18;
}

/* Byte k of the quantization block of `type` that starts at slice offset s. */
static uint8_t synth_block_byte(unsigned type, uint64_t key, uint64_t s, unsigned k) {
    uint64_t o = s + k;
    switch (type) {
    case FO_Q4_K:
        if (k < 4) {
            uint16_t h = fo_synth_scale(synth_hash(key, 1, s + (k & 2)));
            return (uint8_t)(k & 1 ? h >> 8 : h);
        }
        break;
    case FO_Q8_0:
        if (k < 2) {
            uint16_t h = fo_synth_scale(synth_hash(key, 1, s));
            return (uint8_t)(k & 1 ? h >> 8 : h);
        }
        return (uint8_t)(int8_t)((int)((synth_hash(key, 2, o) >> 32) % 255u) - 127);
    case FO_MXFP4:
        if (k == 0) return (uint8_t)(118 + (synth_hash(key, 1, s) >> 32) % 13u);
        break;
    default: /* Q4_0 */
        if (k < 2) {
            uint16_t h = fo_synth_scale(synth_hash(key, 1, s));
            return (uint8_t)(k & 1 ? h >> 8 : h);
        }
        break;
    }
    return (uint8_t)(synth_hash(key, 0, o >> 3) >> (8 * (o & 7)));
}

/* Byte o of the slice (layer, expert) of ownership block `block`, in the
 * reference's slice layout: 32 gate rows, 32 up rows, then the down rows
 * (src/native.h:9-15; transposed for FO_FMT_Q4KT). */
uint8_t fo_synth_byte(const fo_layout *l, uint64_t key, unsigned expert, uint64_t o) {
    int shared = expert == FO_SHARED;
    unsigned gu = shared ? l->shared_gu_type : l->gu_type, dn = shared ? l->shared_down_type : l->down_type;
    uint64_t proj = shared ? l->shared_proj : l->proj;
    if (o < 2 * proj) {
        uint64_t row = fo_row_bytes(gu, l->hidden), rl = (o < proj ? o : o - proj) % row;
        unsigned k = (unsigned)(rl % type_block_bytes(gu));
        return synth_block_byte(gu, key, o - k, k);
    }
    uint64_t od = o - 2 * proj;
    uint64_t drow = (!shared && l->down_transposed) ? fo_row_bytes(dn, l->hidden) : fo_row_bytes(dn, FO_NEURONS);
    unsigned k = (unsigned)(od % drow % type_block_bytes(dn));
    return synth_block_byte(dn, key, o - k, k);
}

void fo_synth_slice(uint8_t *slice, const fo_layout *l, uint64_t seed, unsigned block, unsigned layer,
                    unsigned expert) {
    uint64_t key = fo_synth_key(seed, block, layer, expert);
    uint64_t n = expert == FO_SHARED ? l->shared_slice : l->slice;
    for (uint64_t o = 0; o < n; ++o) slice[o] = fo_synth_byte(l, key, expert, o);
}
