/* fronk_hip.h - C ABI of libfronk_hip.so, the MI355X (gfx950) expert-slice engine.
 *
 * The reference's backend plugin API is the fr_backend vtable
 * (src/backend.h:52-67). Its hot path, run() for expert neuron slices, is
 * implemented here as HIP kernels; fronk_amd/host/hip.c is the drop-in vtable
 * ("hip", next to ref/avx2/neon/metal) that calls these entry points. Only C
 * types cross this boundary: plain pointers, sizes and int return codes that
 * use the reference's FR_* values (src/backend.h:17-18).
 *
 * All calls are synchronous with respect to the host unless noted, and are
 * externally serialized per process like the vtable (src/backend.h:2).
 */
#ifndef FRONK_HIP_H
#define FRONK_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Return codes: the reference's values (src/backend.h:17-18). */
enum { FR_HIP_OK = 0, FR_HIP_INVALID = -1, FR_HIP_STATE = -2, FR_HIP_NUMERIC = -3,
       FR_HIP_IO = -4, FR_HIP_UNSUPPORTED = -5 };

/* Unit formats. LEGACY is the Q4_0 ownership block (src/backend.h:37-50) and
 * NATIVE the lossless GGUF unit (src/native.h:1-15: routed Q4_K gate/up, MXFP4
 * down [H x 32], shared Q8_0). Q4KT, Q8 and MXFP4 are the same unit with every
 * routed projection Q4_K (down stored transposed [32 x H]), Q8_0 or MXFP4. */
enum { FR_HIP_FMT_LEGACY = 0, FR_HIP_FMT_NATIVE = 1, FR_HIP_FMT_Q4KT = 2,
       FR_HIP_FMT_Q8 = 3, FR_HIP_FMT_MXFP4 = 4 };

/* Arithmetic modes of run().
 * F32: fp32 activations, fp32 dot products, fp64 accumulation over experts
 *      and blocks; parity with `ref` (backends/ref.c:124) at 1e-5 rel. L2.
 * F64: fp32 activations, exactly decoded weights, fp64 dot products: the
 *      arithmetic of `ref` (backends/ref.c:57-98) up to summation order.
 * Q8:  `ref-q8` (backends/ref.c:125): x and each slice's h quantized by the
 *      reference quantizer (src/q4.c:37-61), bit-exact, with fp64 dots (on
 *      all-Q4_K units: exact integer dots of x's two int8 digits, summed in
 *      fp64).
 * Q8_256: the AVX2 backend's arithmetic (backends/avx2.c:170-174): x as int8
 *      codes per 256 by quantize8 (avx2.c:184-203, bit-exact), integer dots
 *      times one float scale per block, SiLU in float, h as int8 codes per 32
 *      (quantize8, avx2.c:434), integer down dots times the block scale, the
 *      codes' d and the gate; sums over units in fp64. Native units (Q4_K
 *      gate/up, MXFP4 down, Q8_0 shared expert) and all-Q8_0 units;
 *      requests on legacy Q4_0 blocks run as Q8 (that backend's legacy codes,
 *      avx2.c:83-100, are fr_q8_activation's); other formats return
 *      FR_HIP_UNSUPPORTED. */
enum { FR_HIP_MODE_F32 = 0, FR_HIP_MODE_F64 = 1, FR_HIP_MODE_Q8 = 2, FR_HIP_MODE_Q8_256 = 3 };

/* ggml type ids accepted by the debug decoders (src/native.h:8). */
enum { FR_HIP_Q4_0 = 2, FR_HIP_Q8_0 = 8, FR_HIP_Q4_K = 12, FR_HIP_MXFP4 = 39 };

/* One layer request of 1..8 tokens; the fields of fr_req
 * (src/backend.h:20-25) with the hidden size as a parameter. */
typedef struct {
    unsigned layer, burst, hidden, mode;
    const uint16_t *expert;  /* [burst][10] distinct routed ids < 512 */
    const float *gate;       /* [burst][11], index 10 = shared expert 512 */
    const float *x;          /* [burst][hidden] */
} fr_hip_request;

/* Counters in the spirit of fr_avx2_sample (src/avx2.h:11-15). */
typedef struct {
    uint64_t runs, weight_bytes, hot_allocations;
    unsigned blocks, unique_experts, pairs, grid;
    double last_kernel_ns;
} fr_hip_sample;

/* Device setup and teardown. Replaces the lazy pool setup of load
 * (backends/avx2.c:561-607, backends/metal.m:370-373). Returns
 * FR_HIP_UNSUPPORTED when `device` is not a gfx950 GPU. */
int fr_hip_open(int device);
int fr_hip_close(void);
/* Name of the open device's architecture ("gfx950"), for probe(). */
int fr_hip_probe(int device, char *arch, size_t cap);

/* Copy a whole 48-layer unit to HBM and re-tile it for the kernels
 * (load: src/backend.h:55-61; layout src/native.h:9-21). `len` must equal the
 * unit size of (`hidden`, `format`). */
int fr_hip_upload(unsigned block, const void *unit, uint64_t len, unsigned hidden, unsigned format);
/* Allocate a zero-filled device unit without copying (the slices are then
 * written with fr_hip_refresh). For sparse fixtures and device-side data. */
int fr_hip_reserve(unsigned block, unsigned hidden, unsigned format);
/* Re-read one (layer, expert) slice of a loaded block from `unit`, the
 * borrowed host bytes, so that run() sees later host-side changes
 * (src/native.c:118-130 mutates the unit after load). */
int fr_hip_refresh(unsigned block, const void *unit, unsigned layer, unsigned expert);
/* Measurement data without a host unit (no reference counterpart; the
 * reference's bench fills host units, src/bench.c:279-334): allocate layers
 * [0, layers) of block `block` and fill every slice with seeded synthetic
 * weights, written re-tiled by a device generator. Byte o of slice (layer,
 * expert) in the reference slice layout is a pure function of (seed, block,
 * layer, expert, o): Q4_K d/dmin = fp16(U[1e-3,1e-2]) with uniform nibbles
 * and 6-bit scales, Q8_0 int8 U[-127,127] with an fp16(U[1e-3,1e-2]) scale,
 * MXFP4 E8M0 U[118,130] with uniform codes. run() on a layer >= `layers`
 * returns FR_HIP_STATE. */
int fr_hip_synthetic(unsigned block, unsigned hidden, unsigned format, unsigned layers, uint64_t seed);
/* Free one block's device copy (unload: src/backend.h:62). */
int fr_hip_release(unsigned block);
/* Unit bytes of a (hidden, format) pair, 0 if unsupported. */
uint64_t fr_hip_unit_bytes(unsigned hidden, unsigned format);
/* The device's capacity for units, for the node's share: selection_capacity
 * (src/selection.c:227-244) counts host memory only, while this backend
 * keeps every loaded unit in HBM. Returns in *blocks how many units of
 * (hidden, format) the device holds in its free memory plus the units this
 * engine already holds there, less `reserve` bytes, capped at 20 blocks;
 * *free_bytes is the device's free memory now. No open engine needed. */
int fr_hip_capacity(int device, unsigned hidden, unsigned format, uint64_t reserve, uint64_t *free_bytes,
                    unsigned *blocks);

/* The hot path (run: src/backend.h:63, backends/ref.c:57-98): the plan
 * (routing, gates, x) built on the host and staged into device memory by a
 * copy kernel, one launch over every (expert, owned slice) pair (the decode
 * kernel and its fixed-order reduction, or the layer kernel), y and status
 * back through mapped host memory, one stream wait. A Q8 request whose
 * all-Q4_K units meet a weight the reference rounds in float is repeated on
 * the layer kernel. y receives burst*hidden floats only on success. Request
 * validation is the caller's (backends/ref.c:41-56); this checks shapes. */
int fr_hip_run(const fr_hip_request *req, float *y);

/* Resident-input path for timing: build the plan (and x) into host memory,
 * copy it to device memory the caller owns, then enqueue launches on
 * `stream` (a hipStream_t; NULL = the library stream). The host copy gives
 * the launch shape and, for the decode kernels, the header fields and token
 * table they take as launch arguments; the device copy is what the kernels
 * read otherwise (descriptors, x), so the two must hold the same plan, also
 * when a launch is captured in a graph and replayed. `cap` must be at least
 * fr_hip_plan_bytes(burst, hidden). */
size_t fr_hip_plan_bytes(unsigned burst, unsigned hidden);
int fr_hip_plan(const fr_hip_request *req, void *plan, size_t cap, size_t *used, unsigned *grid);
int fr_hip_launch(const void *host_plan, const void *device_plan, void *stream);
/* Wait for `stream` and copy the last launch's status word and y
 * (burst*hidden floats) to the host. */
int fr_hip_last_output(void *stream, float *y, size_t count, unsigned *status);

/* fr_hip_launch for callers that cannot allocate (no reference counterpart):
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. It calls no allocating routine: the decode kernels' scratch is
 * a static device array of the library (the partials of up to 256 work
 * items, 4.2 MB, held by each GPU the library runs on until the process
 * ends), and y and the status word are device memory the caller passes.
 * Runs plans of one token whose units take the decode kernels
 * (decode_kernel, decode_split_kernel or decode_rows_kernel, then the
 * fixed-order reduction): up to 256 items, which every F32 single-token
 * plan of up to 20 blocks fits (10 routed experts and the shared one);
 * anything else returns FR_HIP_UNSUPPORTED. Enqueued on `stream`
 * (NULL = the library stream); when it completes, *device_status is 0 and
 * device_y holds the hidden outputs, or *device_status has the error bits
 * (FR_NUMERIC cases; device_y is then unspecified). Calls that overlap on
 * one GPU share its static array and race; successive calls need nothing
 * cleared between them. */
int fr_hip_launch_static(const void *host_plan, const void *device_plan, float *device_y, unsigned *device_status,
                         void *stream);

int fr_hip_sample_get(fr_hip_sample *out);

/* Phase times of the last successful fr_hip_run (its kernels ran; an
 * FR_NUMERIC result counts), in ns, after the Metal backend's encode / queue /
 * gpu / return sample (src/metal.h:9-15, backends/metal.m:572-585) and the
 * AVX2 backend's probe timers (backends/avx2.c:38-42):
 *   PLAN     host plan build (routing, gates, x into pinned memory);
 *   ENQUEUE  the launches (plan staging copy kernel, decode kernel and its
 *            reduction, or the layer kernel);
 *   WAIT     from the last launch until y and the status are in host memory
 *            and y is copied out;
 *   GPU      device time from before the staging kernel to after the last
 *            kernel, from two HIP events that are recorded only while
 *            fr_hip_phase_events(1) is in force (they lengthen the call);
 *            0 otherwise;
 *   OVERHEAD TOTAL - GPU;
 *   TOTAL    the whole call.
 * A ref-q8 call repeated on the layer kernel sums both attempts. The host
 * phases are always taken (a few clock reads per call). *runs counts the
 * calls sampled since open. */
enum { FR_HIP_PHASE_PLAN, FR_HIP_PHASE_ENQUEUE, FR_HIP_PHASE_WAIT, FR_HIP_PHASE_GPU, FR_HIP_PHASE_OVERHEAD,
       FR_HIP_PHASE_TOTAL, FR_HIP_PHASES };
int fr_hip_phase_events(int on);
int fr_hip_phase_get(double *ns, uint64_t *runs);

/* Kernel selection for comparison tests and measurements (no reference
 * counterpart). By default a request runs on the first kernel that covers
 * it: the decode kernels (decode_kernel / decode_rows_kernel and their
 * fixed-order reduction), then layer_kernel. FR_HIP_ROUTE_NO_DECODE sends
 * every request to layer_kernel. Bursts of all-Q4_K units whose tokens share
 * experts (10 T >= 2 unique experts) run one unique pair at a time on
 * decode_burst_kernel, other bursts one (token, pair) unit at a time on
 * decode_kernel; FR_HIP_ROUTE_NO_BURST sends every such burst to
 * decode_kernel, FR_HIP_ROUTE_BURST every such burst to decode_burst_kernel. Applies to plans built after the call;
 * FRONK_HIP_NO_DECODE in the environment gives the value at open. */
enum { FR_HIP_ROUTE_NO_DECODE = 2, FR_HIP_ROUTE_NO_BURST = 4, FR_HIP_ROUTE_BURST = 8 };
int fr_hip_route(unsigned flags);

/* Streaming-read probe for the achievable-bandwidth figure (no reference
 * counterpart; the reference reads its own machine's stream rate in
 * backends/metal.m:265-270 and tools/avx2-probe.c:12-30). Enqueues on
 * `stream` one launch of `count` workgroups of `threads` threads (a multiple
 * of 64, at most 1024): workgroup b reads the device byte range
 * (pieces[2b], pieces[2b+1]) = (16-byte aligned address, length < 2^31) with
 * 16-byte loads, `depth` (1, 2, 4 or 8) loads in flight per thread, and
 * stores 16 words to sink[16b..16b+15]. `device_pieces` and `device_sink`
 * are device memory the caller owns. */
int fr_hip_stream_probe(const void *device_pieces, unsigned count, unsigned threads, unsigned depth,
                        void *device_sink, void *stream);

/* Prefill chunk on matrix cores (config "resident node, 512-token prefill").
 * The reference has no multi-token entry beyond run()'s burst of 8: its
 * client cuts longer prompts into bursts (client/fronk_client.h:41-42) and
 * every burst goes through run() (src/backend.h:63, backends/ref.c:57-98).
 * This is fr_hip_run_batch, the extension the hot path's prefill needs: `tokens`
 * tokens of one layer, each with its own routing, in one launch sequence that
 * reads each routed expert's weights once for all of its tokens. Row t of y is
 * run() of token t alone (same validation of ids, FR_NUMERIC rule), within
 * the F32 tolerance. Supported: mode F32, every loaded block FR_HIP_FMT_Q4KT or
 * every loaded block FR_HIP_FMT_NATIVE (the reference's own units: Q4_K
 * gate/up rows, MXFP4 down), the shared expert (gate[t][10] != 0, its Q8_0
 * slices) on any tokens; other formats or a mix return FR_HIP_UNSUPPORTED and
 * the caller uses run(). tokens <= 4096. y receives tokens*hidden floats only
 * on success. */
typedef struct {
    unsigned layer, tokens, hidden, mode;
    const uint16_t *expert;  /* [tokens][10] distinct routed ids < 512 */
    const float *gate;       /* [tokens][11], index 10 = shared expert 512 */
    const float *x;          /* [tokens][hidden] */
} fr_hip_batch;
int fr_hip_run_batch(const fr_hip_batch *req, float *y);
/* Resident-input form of fr_hip_run_batch, like fr_hip_plan/fr_hip_launch:
 * the plan (routing groups and x) is built on the host, copied by the caller
 * to device memory it owns, and launched on `stream`; fr_hip_batch_output
 * waits and reads the status word and y of the last batch launch. */
size_t fr_hip_batch_plan_bytes(unsigned tokens, unsigned hidden);
int fr_hip_batch_plan(const fr_hip_batch *req, void *plan, size_t cap, size_t *used);
int fr_hip_batch_launch(const void *host_plan, const void *device_plan, void *stream);
int fr_hip_batch_output(void *stream, float *y, size_t count, unsigned *status);

/* Launch timing for measurement (no reference counterpart): after
 * fr_hip_timing(n), the next n launches record HIP events on their stream
 * before the main kernel, after it and after the launch's last kernel (a
 * single-token all-Q4_K launch is the decode kernel followed by its
 * fixed-order partial reduction). fr_hip_timing_read waits for them and
 * returns the summed main-kernel and whole-launch times in ms, then stops
 * timing. fr_hip_timing(0) stops without reading. */
int fr_hip_timing(unsigned launches);
int fr_hip_timing_read(double *main_ms, double *total_ms, unsigned *launches);

/* Parity hooks (no reference counterpart): the hot path's own device
 * decoder and quantizer on caller data, for bit-exact checks against the
 * reference's fr_native_dot decode (src/native.c:13-31) and fr_q8_activation
 * (src/q4.c:37-61). `row` is one native row of n weights. */
int fr_hip_debug_dequant(unsigned type, const void *row, unsigned n, float *out);
/* Down matrix of one slice, native bytes, decoded to [hidden][32] floats
 * (element (d, n) = weight of neuron n for output d) for every down format. */
int fr_hip_debug_dequant_down(unsigned format, const void *down, unsigned hidden, float *out);
int fr_hip_debug_quantize(const float *x, unsigned n, float *out);
/* The same quantizer in its register form (q8_regs64: one 64-value group held
 * in one lane's registers), which the single-token Q8 path applies to x;
 * n a multiple of 64. */
int fr_hip_debug_quantize64(const float *x, unsigned n, float *out);
/* The Q8_256 quantizers against the AVX2 backend's quantize8
 * (backends/avx2.c:184-203): group 256 runs the decode kernel's x staging on
 * one token (n a multiple of 256, at most 4096; codes q[n], d[n/256], int16
 * sums s[n/32]); group 32 runs its h quantizer (n = 32; q[32], d[1]; s is not
 * written). */
int fr_hip_debug_quantize8(const float *x, unsigned n, unsigned group, int8_t *q, float *d, int16_t *s);
/* fr_q8_activation as the ref-q8 decode kernels apply it, read back from
 * their LDS: form 0 stages x (n a multiple of 64, at most 4096) as
 * decode_q8_kernel does, form 1 as decode_rows_q8_kernel does (lane-major);
 * each value comes back rebuilt from its two staged digits (s*k + u*r) and
 * sums[n/32] gets the staged exact sum of each 32-value sub-block. Form 2 runs
 * the kernels' h quantizer on n = 32 values (sums unused). A non-finite x
 * gives FR_HIP_NUMERIC, as fr_q8_activation's FR_NUMERIC. */
int fr_hip_debug_quantize_staged(const float *x, unsigned n, unsigned form, float *out, double *sums);
/* The fp32 partials of the last F32 decode launch on the engine's scratch
 * (fr_hip_run or fr_hip_launch): items [first, first + count) of its token-
 * major numbering (a token's (expert, block) units in request order, blocks
 * ascending; split plans: unit * split + part), each as out[item][4096] in
 * output order (columns past the hidden size are the kernel's zeros). For
 * locating a wrong item exactly. */
int fr_hip_debug_partials(unsigned first, unsigned count, float *out);
/* Copy `len` re-tiled device bytes of a block, from byte `offset`. */
int fr_hip_debug_read(unsigned block, uint64_t offset, void *out, uint64_t len);

#ifdef __cplusplus
}
#endif
#endif
