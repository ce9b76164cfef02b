/* hip.c - the "hip" fr_backend: expert neuron slices on an MI355X (gfx950).
 *
 * The backend plugin contract is src/backend.h:52-67; this file is the drop-in
 * next to backends/ref.c, avx2.c, neon.c and metal.m (the same shape as
 * backends/user-template.c), built in the reference tree against its src/
 * headers. All GPU work goes through the C ABI of libfronk_hip.so
 * (include/fronk_hip.h): plain pointers, sizes and FR_* return codes.
 *
 * Semantics kept from the reference:
 *   probe   NULL -> FR_INVALID; hw_probe failure -> FR_IO; no gfx950 GPU ->
 *           FR_UNSUPPORTED before anything that can fault (backends/avx2.c:76-82).
 *   load    range, NULL and length checks -> FR_INVALID, occupied slot ->
 *           FR_STATE (backends/user-template.c:17-21); the length selects the
 *           native (src/native.h:15) or legacy Q4_0 (src/backend.h:37-50) unit.
 *           The device is opened at the first load (backends/avx2.c:602-607).
 *           Unlike ref/avx2, the bytes are copied to HBM and re-tiled, because
 *           the kernels read HBM, not host memory.
 *   run     ref's validation order (backends/ref.c:41-56), FR_STATE when nothing
 *           is loaded, *out replaced completely on success and untouched on any
 *           failure (src/backend.h:4-5), no allocation.
 *   bench   fr_bench_execute_backend (backends/user-template.c:93).
 *   self_test  FR_STATE when a block is loaded; the golden corpus, then the
 *           native self-test (backends/avx2.c:773-777).
 *   fr_hip_backend_close  the bench's close hook (src/bench.c:265-278).
 * A second table, "hip-q8", is this backend with the ref-q8 arithmetic
 * (backends/ref.c:66,85: x and h through fr_q8_activation, fp64 sums), the
 * counterpart of the reference's ref / ref-q8 pair (backends/ref.c:124-125).
 * A third, "hip-q8-256", runs the AVX2 backend's arithmetic (x and h through
 * its quantize8, backends/avx2.c:184-203, integer dots; FR_HIP_MODE_Q8_256).
 * The tables share the device and the loaded blocks.
 * During self_test, load only reserves device memory and run copies the
 * slices a request references from the borrowed bytes first: the corpus
 * fixtures are sparse multi-GB units, and the native self-test corrupts the
 * host bytes after load and expects FR_NUMERIC (src/native.c:118-130).
 */
#include "backend.h"
#include "bench.h"
#include "native.h"
#include "vectors.h"

#include <fenv.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include "fronk_hip.h"
#include "hip.h"

static const unsigned char *unit[FR_BLOCKS];   /* borrowed until unload */
static int opened;
static int coherent;
static float result[FR_MAX_BURST][FR_HIDDEN];

static int loaded(void) {
    for (unsigned b = 0; b < FR_BLOCKS; ++b)
        if (unit[b]) return 1;
    return 0;
}

static int probe(fr_hwinfo *out) {
    if (!out) return FR_INVALID;
    fr_hwinfo hw;
    if (hw_probe(&hw)) return FR_IO;
    char arch[32] = "";
    if (fr_hip_probe(0, arch, sizeof(arch)) != FR_HIP_OK) return FR_UNSUPPORTED;
    snprintf(hw.gpu, sizeof(hw.gpu), "AMD Instinct (%s)", arch);
    *out = hw;
    return FR_OK;
}

static int load(int b, const void *data, size_t len) {
    if (b < 0 || b >= FR_BLOCKS || !data) return FR_INVALID;
    unsigned format;
    if (len == FR_NATIVE_BLOCK_BYTES) format = FR_HIP_FMT_NATIVE;
    else if (len == FR_WEIGHT_BLOCK_BYTES) format = FR_HIP_FMT_LEGACY;
    else return FR_INVALID;
    if (unit[b]) return FR_STATE;
    if (!opened) {
        int rc = fr_hip_open(0);
        if (rc) return rc;
        opened = 1;
    }
    int rc = coherent ? fr_hip_reserve((unsigned)b, FR_HIDDEN, format)
                      : fr_hip_upload((unsigned)b, data, len, FR_HIDDEN, format);
    if (rc) return rc;
    unit[b] = data;
    return FR_OK;
}

static int unload(int b) {
    if (b < 0 || b >= FR_BLOCKS) return FR_INVALID;
    if (!unit[b]) return FR_STATE;
    int rc = fr_hip_release((unsigned)b);
    unit[b] = NULL;
    return rc;
}

static int validate(const fr_req *r) {
    if (!r || r->layer >= FR_LAYERS || r->burst < 1 || r->burst > FR_MAX_BURST || fegetround() != FE_TONEAREST)
        return FR_INVALID;
    for (unsigned t = 0; t < r->burst; ++t) {
        for (unsigned e = 0; e < FR_ACTIVE_ROUTED; ++e) {
            if (r->expert[t][e] >= FR_ROUTED_EXPERTS) return FR_INVALID;
            for (unsigned k = 0; k < e; ++k)
                if (r->expert[t][k] == r->expert[t][e]) return FR_INVALID;
        }
        for (unsigned e = 0; e < FR_ACTIVE_EXPERTS; ++e) {
            if (!isfinite(r->gate[t][e])) return FR_NUMERIC;
            if (r->gate[t][e] < 0) return FR_INVALID;
        }
        for (unsigned d = 0; d < FR_HIDDEN; ++d)
            if (!isfinite(r->x[t][d])) return FR_NUMERIC;
    }
    return FR_OK;
}

/* Copy every slice the request references (routed ids of every token, the
 * shared expert when a gate selects it) from the borrowed bytes. */
static int refresh_referenced(const fr_req *r) {
    unsigned char seen[FR_EXPERTS];
    memset(seen, 0, sizeof(seen));
    for (unsigned t = 0; t < r->burst; ++t) {
        for (unsigned e = 0; e < FR_ACTIVE_ROUTED; ++e) seen[r->expert[t][e]] = 1;
        if (r->gate[t][FR_ACTIVE_ROUTED] != 0) seen[FR_SHARED_EXPERT] = 1;
    }
    for (unsigned b = 0; b < FR_BLOCKS; ++b) {
        if (!unit[b]) continue;
        for (unsigned id = 0; id < FR_EXPERTS; ++id) {
            if (!seen[id]) continue;
            int rc = fr_hip_refresh(b, unit[b], r->layer, id);
            if (rc) return rc;
        }
    }
    return FR_OK;
}

static int run_mode(const fr_req *r, fr_part *out, unsigned mode) {
    if (!out) return FR_INVALID;
    int rc = validate(r);
    if (rc) return rc;
    if (!loaded()) return FR_STATE;
    if (coherent && (rc = refresh_referenced(r))) return rc;
    fr_hip_request q = {r->layer, r->burst, FR_HIDDEN, mode, &r->expert[0][0], &r->gate[0][0], &r->x[0][0]};
    rc = fr_hip_run(&q, &result[0][0]);
    if (rc) return rc;
    out->layer = r->layer;
    out->burst = r->burst;
    memcpy(out->y, result, (size_t)r->burst * sizeof(result[0]));
    memset(out->y[r->burst], 0, (size_t)(FR_MAX_BURST - r->burst) * sizeof(out->y[0]));
    return FR_OK;
}

static int run(const fr_req *r, fr_part *out) { return run_mode(r, out, FR_HIP_MODE_F32); }
static int run_q8(const fr_req *r, fr_part *out) { return run_mode(r, out, FR_HIP_MODE_Q8); }
static int run_q8_256(const fr_req *r, fr_part *out) { return run_mode(r, out, FR_HIP_MODE_Q8_256); }

static int bench(int burst_max, fr_costmodel *out) { return fr_bench_execute_backend(&fr_hip, burst_max, out); }
static int bench_q8(int burst_max, fr_costmodel *out) { return fr_bench_execute_backend(&fr_hip_q8, burst_max, out); }
static int bench_q8_256(int burst_max, fr_costmodel *out) {
    return fr_bench_execute_backend(&fr_hip_q8_256, burst_max, out);
}

static int check(const fr_backend *b, const char *dir) {
    if (loaded()) return FR_STATE;
    coherent = 1;
    int rc = fr_vectors_check(b, dir, &fr_backend_tolerance, NULL);
    if (!rc) rc = fr_native_self_test(b);
    coherent = 0;
    return rc;
}
static int self_test(const char *dir) { return check(&fr_hip, dir); }
static int self_test_q8(const char *dir) { return check(&fr_hip_q8, dir); }
static int self_test_q8_256(const char *dir) { return check(&fr_hip_q8_256, dir); }

const fr_backend fr_hip = {"hip", probe, load, unload, run, bench, self_test};
const fr_backend fr_hip_q8 = {"hip-q8", probe, load, unload, run_q8, bench_q8, self_test_q8};
const fr_backend fr_hip_q8_256 = {"hip-q8-256", probe, load, unload, run_q8_256, bench_q8_256, self_test_q8_256};

/* The bench's backend_close hook (src/bench.c:265-278), like fr_avx2_close
 * (backends/avx2.c:718): FR_STATE while a block is loaded, otherwise release
 * the device so that the next load opens it afresh. */
int fr_hip_backend_close(void) {
    if (loaded()) return FR_STATE;
    if (!opened) return FR_OK;
    int rc = fr_hip_close();
    if (!rc) opened = 0;
    return rc;
}

#ifdef FR_HIP_MODULE
/* Module form (tools/backend-module.py): the table under the name the module
 * registry expects (src/backend.c:56-58). */
const fr_backend fr_module_hip = {"hip", probe, load, unload, run, bench, self_test};
#endif
