/* fronk_oracle.h - CPU restatement of the reference's expert-slice algorithm.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may call it; the product
 * (fronk_amd/, include/) never links, loads or calls anything under oracle/.
 *
 * Every function restates one reference function (file:line given at the
 * definition in fronk_oracle.c). The hidden size H is a run-time parameter
 * (the reference fixes it at 2560, src/model.h:16); the down projection may be
 * stored in the reference's native [H x 32] orientation or transposed
 * [32 x H] (a layout the reference does not have; see FO_FMT_Q4KT).
 *
 * Parity pins (each is a test under tests/):
 *   fo_f16            exhaustive 65,536 codes vs the IEEE binary16 closed form
 *   fo_q4_dot         nibble-basis KATs + the 8 committed golden partials
 *   fo_q8_activation  KATs of tests/test_q4.c:39-57 + oracle/_ref byte compare
 *   fo_quantize8      closed-form KATs (ties, saturation, zero group)
 *   fo_native_dot     256-lane Q4_K basis, MXFP4 LUT/sign/order, Q8_0 byte KATs
 *   fo_ref_run        golden corpus (byte-identical regeneration), analytic
 *                     SiLU(1) closed forms, oracle/_ref on native fixtures,
 *                     brute-force numpy dense matmul for the H=4096 formats
 *   fo_compare        metric edge cases of tests/test_backend.c:162-184
 */
#ifndef FRONK_ORACLE_H
#define FRONK_ORACLE_H
#include <stddef.h>
#include <stdint.h>

enum { FO_OK = 0, FO_INVALID = -1, FO_STATE = -2, FO_NUMERIC = -3, FO_IO = -4 };

/* Geometry that does not depend on H (src/model.h:13-27). */
enum { FO_LAYERS = 48, FO_ROUTED = 512, FO_EXPERTS = 513, FO_SHARED = 512,
       FO_ACTIVE_ROUTED = 10, FO_ACTIVE = 11, FO_NEURONS = 32, FO_BLOCKS = 20,
       FO_MAX_BURST = 8, FO_MAX_HIDDEN = 4096 };

/* ggml type ids used by the reference (src/native.h:8) plus legacy Q4_0. */
enum { FO_Q4_0 = 2, FO_Q8_0 = 8, FO_Q4_K = 12, FO_MXFP4 = 39 };

/* Unit formats. LEGACY and NATIVE are the reference's two block layouts
 * (src/backend.h:37-50, src/native.h:1-15). The other three carry the
 * measurement configurations at H=4096:
 *   Q4KT  routed gate/up Q4_K [32 x H], down Q4_K stored transposed [32 x H]
 *   Q8    routed gate/up Q8_0 [32 x H], down Q8_0 [H x 32]
 *   MXFP4 routed gate/up MXFP4 [32 x H], down MXFP4 [H x 32]
 * The shared expert (id 512) is Q8_0 x 3 in every format but LEGACY. */
enum { FO_FMT_LEGACY = 0, FO_FMT_NATIVE = 1, FO_FMT_Q4KT = 2, FO_FMT_Q8 = 3, FO_FMT_MXFP4 = 4 };

typedef struct {
    unsigned hidden, format;
    unsigned gu_type, down_type, down_transposed;   /* routed slice */
    unsigned shared_gu_type, shared_down_type;
    uint64_t gu_row, down_row;         /* bytes per gate/up row, per stored down row */
    uint64_t proj, down, slice;        /* routed projection (32 rows), down, slice */
    uint64_t shared_proj, shared_down, shared_slice;
    uint64_t layer, block;             /* bytes per layer, per 48-layer unit */
} fo_layout;

typedef struct {
    unsigned layer, burst, hidden;
    uint16_t expert[FO_MAX_BURST][FO_ACTIVE_ROUTED];
    float gate[FO_MAX_BURST][FO_ACTIVE];
    float x[FO_MAX_BURST][FO_MAX_HIDDEN];
} fo_req;

float fo_f16(uint16_t bits);
uint64_t fo_row_bytes(unsigned type, unsigned n);
int fo_layout_get(unsigned hidden, unsigned format, fo_layout *out);
uint64_t fo_slice_offset(const fo_layout *l, unsigned layer, unsigned expert);

int fo_q4_dot(const uint8_t *q, const float *x, size_t n, double *out);
int fo_q8_activation(const float *x, float *out, size_t n);
void fo_quantize8(const float *x, unsigned n, unsigned group, int8_t *q, float *d, int16_t *s);
int fo_native_dot(const uint8_t *p, unsigned type, const float *x, unsigned n, double *out);
/* Element j of a row of `type`, decoded exactly as the dot products do. */
float fo_decode(const uint8_t *row, unsigned type, unsigned j);
int fo_dequant_row(const uint8_t *row, unsigned type, unsigned n, float *out);

/* ref / ref-q8 run() over one request. blocks[b] is NULL when block b is not
 * loaded. y must hold burst*hidden floats. Returns FO_* codes in the
 * reference's order; y is written only on success. */
int fo_ref_run(const uint8_t *const blocks[FO_BLOCKS], unsigned format, int q8,
               const fo_req *req, float *y);

int fo_compare(const float *ref, const float *actual, size_t n, double out[3]);
int fo_conforms(const double e[3], const double limit[3]);

/* Golden corpus recipe at H=2560, LEGACY format (src/vectors.c:12-82). */
int fo_vector_request(unsigned index, fo_req *req, uint32_t *mask, char name[16]);
int fo_vector_fill(unsigned index, uint8_t *const blocks[FO_BLOCKS], char digest[65]);
int fo_vector_format(unsigned index, const fo_req *req, uint32_t mask, const char *digest,
                     const float *y, char *out, size_t cap, size_t *len);

/* Native fixture recipe (src/native.c:39-65) for any hidden size and format. */
uint32_t fo_lcg(uint32_t *seed);
void fo_fill_slice(uint8_t *slice, const fo_layout *l, unsigned expert, uint32_t *seed);

/* Synthetic measurement weights (distributions in fronk_oracle.c): byte o of
 * slice (layer, expert) of ownership block `block`, reference slice layout. */
uint64_t fo_synth_key(uint64_t seed, unsigned block, unsigned layer, unsigned expert);
uint16_t fo_synth_scale(uint64_t h);
uint8_t fo_synth_byte(const fo_layout *l, uint64_t key, unsigned expert, uint64_t o);
void fo_synth_slice(uint8_t *slice, const fo_layout *l, uint64_t seed, unsigned block, unsigned layer,
                    unsigned expert);

void fo_sha256(const void *data, size_t len, uint8_t out[32]);
#endif
