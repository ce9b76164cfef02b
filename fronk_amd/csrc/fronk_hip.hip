// fronk_hip.hip - MI355X (gfx950) expert neuron-slice engine behind a C ABI.
//
// One run() of the reference backend contract (src/backend.h:63) is ONE
// kernel launch covering every (expert, owned 32-neuron slice) pair of a
// layer request. The launch is a list of workgroup tasks, dispatched in
// block-index order:
//
//   phase A  (pair, 8 neurons): the pair's gate and up rows are streamed
//            once from HBM, dequantized in registers and dotted with the
//            activation staged in LDS, one wavefront per row; a DPP/shuffle
//            tree reduces each row; h = SiLU(a)*u goes to a small device
//            buffer and a per-pair counter is released.
//   phase B  (group of pairs, 256 output dims): waits (bounded) until every
//            pair of its group has all 32 h values, then streams the down
//            weights of the group and accumulates gate*W_down*h for its 256
//            output dims in fp64; the group partial goes to scratch.
//   reduce   the last phase-B task of each 256-dim range (atomic ticket)
//            sums the group partials in a fixed order and writes y.
//
// No fp32 atomics touch y: the result is bit-reproducible run to run and a
// token's bits do not depend on which other tokens share the burst beyond
// fp64 summation order. Reference semantics: backends/ref.c:57-98.
#include <hip/hip_runtime.h>

#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <cmath>
#include <type_traits>
#include <vector>

#include "fronk_hip.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kNeurons = 32;
constexpr int kMaxBurst = 8;
constexpr int kBlocks = 20;
constexpr int kLayers = 48;
constexpr int kRouted = 512;
constexpr int kShared = 512;
constexpr int kMaxUnique = kMaxBurst * 10 + 1;
constexpr int kMaxPairs = kMaxUnique * kBlocks;
constexpr int kCols = 256;            // output dims per phase-B task
constexpr int kMaxHidden = 4096;
constexpr int kMaxRanges = kMaxHidden / kCols;
constexpr int kLdsLimit = 64 * 1024;
constexpr uint32_t kSpinLimit = 1u << 16;   // about 0.1 s of polling
constexpr int kDecodeThreads = 512;         // decode kernel: 8 wavefronts
constexpr int kDecodeWaves = kDecodeThreads / 64;
constexpr int kDecodeGridMax = 256;         // decode workgroups (one per CU at most)

// Status bits of the output word.
constexpr uint32_t kErrScale = 1;     // referenced non-finite scale
constexpr uint32_t kErrRange = 2;     // a, u, h or y outside fp32
constexpr uint32_t kErrTimeout = 4;   // dependency wait exceeded its bound

enum : uint8_t { TQ4_0 = 2, TQ8_0 = 8, TQ4_K = 12, TMXFP4 = 39, TQ4_KT = 140, TQ4_KM = 141 };
// TQ4_KM: the routed Q4_K gate/up rows of a pair in matrix-core tiles (see
// the re-tiled layouts); it decodes as TQ4_K once loaded.
template <int GU> constexpr int kAs = GU == TQ4_KM ? TQ4_K : GU;
enum { MODE_F32 = 0, MODE_F64 = 1, MODE_Q8 = 2, MODE_Q8_256 = 3 };

struct PairDesc {            // one (expert, block) slice of the request
  uint64_t slice;            // device address of the re-tiled slice
  uint32_t proj;             // bytes of the 32 gate rows (= up offset)
  uint8_t gu, dn, tmask, pad;
  float gate[kMaxBurst];     // per-token expert weight (0 when not routed)
};
static_assert(sizeof(PairDesc) == 48, "pair layout");

struct GroupDesc {
  uint16_t first, count;
  uint8_t dn, pad[3];
};
static_assert(sizeof(GroupDesc) == 8, "group layout");

struct PlanHeader {
  uint32_t hidden, burst, mode, npairs;
  uint32_t ngroups, nranges, ntA, ntB;
  uint32_t nn, tchunk, pairs_off, groups_off;
  uint32_t x_off, total, gmax, lds;
  uint32_t kind, grid, tpw, pad;   // kernel (KIND_*), its grid, decode pairs per workgroup
};
static_assert(sizeof(PlanHeader) == 80, "header layout");

// Which kernel a plan runs: the two-phase layer kernel, or the decode
// kernel for all-Q4_K units with the transposed down (F32, routed experts
// only), whose work list is (token, pair) units, token-major, each with its
// own partial.
enum : uint32_t { KIND_LAYER = 0, KIND_DECODE = 1, KIND_DECODE_ROWS = 2, KIND_DECODE_SPLIT = 3, KIND_DECODE_BURST = 4 };
// A decode plan's items (work-list entries with a partial each): one per
// unit, or `split` (2 or 4) per unit for KIND_DECODE_SPLIT.
constexpr int kMaxDecodeItems = 2048;
// A decode plan's token table (at groups_off): token t's units.
struct DecodeToken {
  uint32_t first, count;
};
constexpr int kDecodeUnitsPerToken = 11 * kBlocks;   // 10 routed experts and the shared one
// Decode plans' work lists: every (token, pair) unit of a full burst fits,
// shared expert included.
constexpr int kMaxDecodeUnits = kMaxBurst * kDecodeUnitsPerToken;
constexpr int kMaxPlanPairs = kMaxDecodeUnits > kMaxPairs ? kMaxDecodeUnits : kMaxPairs;
static_assert(kMaxDecodeUnits <= kMaxDecodeItems, "a full burst's unit partials fit");

struct Scratch {
  uint32_t* done;            // [2][kMaxPairs] phase-A wave completions per pair
  uint32_t* fin;             // [2][kMaxRanges] phase-B completions per range
  float* hbuf;               // [kMaxPairs][8][32]
  double* partial;           // [groups][burst][hidden]
  uint32_t* out;             // [2][out_words]: status, pad x3, y
  float* wgpart;             // decode unit partials, [kMaxHidden/16][ustride][16] (partial_index)
  uint32_t* bar;             // [2]: decode workgroups past their partial store
  uint32_t out_words;
  uint32_t parity;
  uint32_t ustride;          // units per position block of wgpart
  // Set by fr_hip_launch_static, null otherwise: the caller's status word
  // and y, and the decode kernels' error word in the static scratch array.
  uint32_t* ystat;
  float* yout;
  uint32_t* dstat;
  // Set by fr_hip_run on the decode path, null otherwise: one status word
  // per decode_reduce workgroup in mapped host memory (yout is then mapped
  // host memory too, and dstat a device word of the engine).
  uint32_t* hstat;
  // Decode launches: the plan header's fields and token table, copied from
  // the host plan (launch_decode). Kernel arguments are the first memory a
  // workgroup reads, so its pair descriptor and x are requested one
  // dependent load earlier than through the device plan's header, and
  // decode_reduce's partials two.
  struct {
    uint32_t hidden, burst, npairs, tpw, pairs_off, groups_off, x_off, pad;
    DecodeToken tok[kMaxBurst];
  } A;
};

// ------------------------------------------------------------ scalars

__device__ __forceinline__ float half_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
__device__ __forceinline__ bool half_bad(uint32_t bits) { return (bits & 0x7c00u) == 0x7c00u; }
// half_bad of both halves of w, as bits to OR together over a loop: bit 15
// (31) of the result is set iff the low (high) half has the all-ones
// exponent (e + 0x400 reaches 0x8000 only for e = 0x7c00, and the low
// half's sum never carries into the high half).
constexpr uint32_t kHalfBadBits = 0x80008000u;
__device__ __forceinline__ uint32_t half_bad_bits(uint32_t w) { return (w & 0x7c007c00u) + 0x04000400u; }

// 2^(e-127) for an E8M0 exponent 0..254; e = 0 is the subnormal 2^-127.
__device__ __forceinline__ float e8m0(uint32_t e) {
  return __uint_as_float(e ? e << 23 : 0x00400000u);
}
// An MXFP4 block (E8M0 exponent e, its 32 codes in q) holding a weight that
// the reference decodes to a non-finite value (src/native.c:23-27: the fp32
// product 2^(e-127) * code value, which run() turns into FR_NUMERIC): e = 255,
// a code of magnitude >= 2 (codes with bit 2 set: 2, 3, 4, 6) at e = 254,
// where 2 * 2^127 = 2^128 overflows, or of magnitude >= 4 (bits 2 and 1 set:
// 4, 6) at e = 253.
__device__ __forceinline__ bool mx_block_bad(uint32_t e, const uint4& q) {
  const uint32_t ge2 = (q.x | q.y | q.z | q.w) & 0x44444444u;
  const uint32_t ge4 = ((q.x & (q.x >> 1)) | (q.y & (q.y >> 1)) | (q.z & (q.z >> 1)) | (q.w & (q.w >> 1))) & 0x22222222u;
  return e == 255u || (e == 254u && ge2 != 0u) || (e == 253u && ge4 != 0u);
}
// mx_block_bad behind a wave-wide screen for the hot loops: only exponents
// 253..255 can make a block bad, so the code test runs (for the whole wave)
// only when some lane holds such an exponent.
__device__ __forceinline__ bool mx_blocks_bad(uint32_t e0, const uint4& q0, uint32_t e1, const uint4& q1) {
  if (__builtin_expect(__ballot((e0 > e1 ? e0 : e1) >= 253u) == 0, 1)) return false;
  return mx_block_bad(e0, q0) || mx_block_bad(e1, q1);
}

// Two OCP E2M1 codes (byte b of v: low nibble first) -> floats times
// `scale`, with the gfx950 conversion instruction. The products are exact
// (E2M1 values have two significant bits, scales are powers of two, the
// subnormal 2^-127 included); code 8 yields -0, the reference table +0
// (src/native.c:9), which only the exact decoders normalize.
__device__ __forceinline__ float2 fp4_pair(uint32_t v, float scale, int b) {
  switch (b) {
    case 0: { auto r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, scale, 0); return make_float2(r[0], r[1]); }
    case 1: { auto r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, scale, 1); return make_float2(r[0], r[1]); }
    case 2: { auto r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, scale, 2); return make_float2(r[0], r[1]); }
    default: { auto r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, scale, 3); return make_float2(r[0], r[1]); }
  }
}

// Q4_K 6-bit scale/min of group g from the 12 packed bytes s0|s1|s2
// (src/native.c:14-19).
// Both cases are computed and one is selected, so that lanes holding
// different groups do not diverge.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t g,
                                              uint32_t& sc, uint32_t& mi) {
  const uint32_t k = 8 * (g & 3u);
  const uint32_t a0 = s0 >> k, a1 = s1 >> k, a2 = s2 >> k;
  const uint32_t sc_hi = (a2 & 15u) | ((a0 >> 2) & 48u);         // low 4 bits | top 2 bits of byte g-4
  const uint32_t mi_hi = ((a2 >> 4) & 15u) | ((a1 >> 2) & 48u);
  sc = g < 4 ? a0 & 63u : sc_hi;
  mi = g < 4 ? a1 & 63u : mi_hi;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Full-wave sum with DPP: quad butterflies, two rotations inside each
// 16-lane row, then the four row totals read as scalars. The result is
// wave-uniform and the association order is fixed.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  uint64_t b = __builtin_bit_cast(uint64_t, v);
  uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
  uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowRor4 = 0x124, kRowRor8 = 0x128, kRowHalfMirror = 0x141;

__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f<kQuadXor1>(v);
  v += dpp_f<kQuadXor2>(v);
  v += dpp_f<kRowRor4>(v);
  v += dpp_f<kRowRor8>(v);
  return v;
}
__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_total(float v) {
  v = row_sum(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  uint64_t b = __builtin_bit_cast(uint64_t, v);
  uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_total(double v) {
  v += dpp_d<kQuadXor1>(v);
  v += dpp_d<kQuadXor2>(v);
  v += dpp_d<kRowRor4>(v);
  v += dpp_d<kRowRor8>(v);
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// Sum over each aligned group of 8 lanes (quad butterflies + half-row mirror).
__device__ __forceinline__ float oct_sum(float v) {
  v += dpp_f<kQuadXor1>(v);
  v += dpp_f<kQuadXor2>(v);
  v += dpp_f<kRowHalfMirror>(v);
  return v;
}

__device__ __forceinline__ void flag(uint32_t* status, uint32_t bit) {
  __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-workgroup publication without cache-maintenance fences. On gfx950
// an agent-scope release writes back the whole L2 of the XCD and an acquire
// invalidates it (measured: ~100 us per 44 MB call when every wave does it).
// Shared values are instead stored with device-coherent (sc1) stores, the
// writing wave drains its memory counter, and only then bumps a relaxed
// counter (an atomic performed at the device coherence point). Readers poll
// the counter relaxed and load the values with device-coherent loads; they
// touch a value's line only after its counter says it is complete.
__device__ __forceinline__ void drain_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
template <typename T>
__device__ __forceinline__ void put(T* p, T v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <typename T>
__device__ __forceinline__ T get(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t bump(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Byte k of v as a float: one v_cvt_f32_ubyte<k> when v holds four nibbles
// already masked to their bytes.
__device__ __forceinline__ float ub(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xffu); }
// The low and high nibbles of the four bytes of v, each in its own byte. The
// AND is opaque to the optimizer, which would otherwise fold it into the byte
// extraction and emit a bit-field extract per nibble.
__device__ __forceinline__ uint32_t nib_lo(uint32_t v) {
  uint32_t r;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(v));
  return r;
}
__device__ __forceinline__ uint32_t nib_hi(uint32_t v) {
  uint32_t r;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(v >> 4));
  return r;
}
// Bytes 2h and 2h+1 of v, each holding a nibble value q in 0..15, as two
// floats q * 2^-9 in one conversion: an FP8 E4M3 byte below 16 is q * 2^-9
// exactly (subnormal below 8, exponent 1 from 8 to 15, spacing 2^-9 in both).
// Callers fold the 2^9 into a scale; a power of two commutes with rounding,
// so the products and sums are those of the unscaled nibbles.
constexpr float kFp8Nibble = 512.f;   // 2^9
template <bool H>
__device__ __forceinline__ float2 nib_pair(uint32_t v) {
  const auto r = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, H);
  return make_float2(r[0], r[1]);
}

// Weight and plan addresses arrive as 64-bit integers, so the compiler sees
// generic pointers and would emit FLAT loads; a FLAT load also counts against
// the LDS/scalar counter, which makes every LDS wait and barrier wait for all
// outstanding weight loads. These go through the global address space.
template <typename T>
__device__ __forceinline__ T gld(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
  const u32x4 v = gld<u32x4>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(const uint8_t* p) {
  const u32x2 v = gld<u32x2>(p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// fr_q8_activation on n <= 64 values held one per lane... here: a whole
// group in registers of one thread (src/q4.c:37-61).
__device__ void q8_group(float* v, int n) {
  float max = 0.f;
  for (int j = 0; j < n; ++j) max = fmaxf(max, fabsf(v[j]));
  float scale = max / 127.0f;
  if (scale == 0.f) {
    for (int j = 0; j < n; ++j) v[j] = 0.f;
    return;
  }
  float inv = 127.0f / max;
  bool finite_inv = isfinite(inv);
  for (int j = 0; j < n; ++j) {
    float q = finite_inv ? v[j] * inv : (v[j] / max) * 127.0f;
    q = rintf(q);
    q = fminf(fmaxf(q, -127.f), 127.f);
    double back = (double)q * (double)scale;
    back = fmin(fmax(back, -(double)FLT_MAX), (double)FLT_MAX);
    v[j] = (float)back;
  }
}

// fr_q8_activation of one 64-value group held in registers (src/q4.c:37-61).
__device__ __forceinline__ void q8_regs64(float4* x4) {
  float max = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    max = fmaxf(fmaxf(fmaxf(max, fabsf(x4[i].x)), fmaxf(fabsf(x4[i].y), fabsf(x4[i].z))), fabsf(x4[i].w));
  const float scale = max / 127.0f;
  const float inv = 127.0f / max;
  const bool zero = scale == 0.f, finite_inv = isfinite(inv);
  auto q = [&](float v) {
    float r = finite_inv ? v * inv : (v / max) * 127.0f;
    r = fminf(fmaxf(rintf(r), -127.f), 127.f);
    double back = fmin(fmax((double)r * (double)scale, -(double)FLT_MAX), (double)FLT_MAX);
    return zero ? 0.f : (float)back;
  };
#pragma unroll
  for (int i = 0; i < 16; ++i) x4[i] = make_float4(q(x4[i].x), q(x4[i].y), q(x4[i].z), q(x4[i].w));
}

// ------------------------------------------------- re-tiled row layouts
//
// Gate/up rows (n = hidden columns, nch = n/64 lane chunks of 64 columns):
//  Q4_K : [2 parts][nch][16 B] quants (bytes 0-15 / 16-31 of each 32-byte
//         chunk of a super-block), then [n/256][16 B] super-block headers.
//  Q8_0 : [4 parts][nch][16 B] int8, then [nch][2 x fp16] scales.
//  MXFP4: [2 parts][nch][16 B] codes, then [nch][2 B] exponents.
//  Q4_0 : [2 parts][nch][16 B] nibbles, then [nch][2 x fp16] scales.
// Lane c reads its 64 columns with 16-byte loads; 64 lanes read contiguous
// 1 KB runs. Same byte count as the native row (the permutation is lossless).
//
// Q4_K gate/up of the transposed-down format (TQ4_KM), the 64 rows of a pair
// together: row-block rb (0..3) holds rows i = 0..7 gate and 8..15 up of
// neurons 8rb + i%8. Per super-block sb: [4 rb][16 rows][16 B] headers
// (1 KB), then [4 rb][2 parts][64 lanes][16 B] nibbles (8 KB). Lane
// l = 16kg + i of part p holds sub-block 4p + kg of row i: its 32 values in
// 4 words, word u having positions 8u..8u+3 in the low nibbles of its bytes
// and 8u+4..8u+7 in the high nibbles. Lane l of part p is then the int8 A
// operand of two 16x16x64 matrix products (row i, k = 16kg..16kg+15) once
// each word is split into its low and high nibbles.

// Decode the lane's 64 columns of a gate/up row exactly as the reference
// decodes each weight (src/native.c:13-31, src/q4.c:29-31). Used by the
// fp64 modes and by the debug decoder; returns false on a non-finite scale.
// The lane's raw bytes of one gate/up row: quants and the scale words.
struct LaneRaw {
  uint4 q[4];
  uint4 h;
};

template <int type>
__device__ __forceinline__ void load_raw(const uint8_t* row, int nch, int c, LaneRaw& r) {
  if (type == TQ4_K) {
    r.q[0] = ld16(row + 16 * c);
    r.q[1] = ld16(row + 16 * nch + 16 * c);
    r.h = ld16(row + 32 * nch + 16 * (c >> 2));
  } else if (type == TQ8_0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) r.q[p] = ld16(row + 16 * nch * p + 16 * c);
    r.h.x = gld<uint32_t>(row + 64 * nch + 4 * c);
  } else if (type == TMXFP4) {
    r.q[0] = ld16(row + 16 * c);
    r.q[1] = ld16(row + 16 * nch + 16 * c);
    r.h.x = gld<uint16_t>(row + 32 * nch + 2 * c);
  } else {
    r.q[0] = ld16(row + 16 * c);
    r.q[1] = ld16(row + 16 * nch + 16 * c);
    r.h.x = gld<uint32_t>(row + 32 * nch + 4 * c);
  }
}

// Row (k = 0 gate, 1 up; neuron n) of a TQ4_KM pair, lane chunk c, in the
// TQ4_K lane form of load_raw: the two 16-byte sub-block runs of chunk c are
// merged back into the reference's 32-byte chunk (byte i: low nibble position
// i of the first sub-block, high nibble position i of the second).
__device__ __forceinline__ void load_km(const uint8_t* slice, int k, unsigned n, int c, LaneRaw& r) {
  const unsigned sb = (unsigned)c >> 2, rb = n >> 3, i = 8 * k + (n & 7), s0 = 2 * ((unsigned)c & 3);
  const uint8_t* blk = slice + 9216 * sb;
  r.h = ld16(blk + 16 * (16 * rb + i));
  const uint8_t* nib = blk + 1024 + 2048 * rb + 1024 * (s0 >> 2) + 16 * i;
  const uint4 a = ld16(nib + 16 * 16 * (s0 & 3)), b = ld16(nib + 16 * 16 * ((s0 & 3) + 1));
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    o[2 * u] = (aw[u] & 0x0f0f0f0fu) | ((bw[u] & 0x0f0f0f0fu) << 4);
    o[2 * u + 1] = ((aw[u] >> 4) & 0x0f0f0f0fu) | (bw[u] & 0xf0f0f0f0u);
  }
  r.q[0] = make_uint4(o[0], o[1], o[2], o[3]);
  r.q[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// Gate (k = 0) or up row of neuron n of a pair for lane chunk c.
template <int GU>
__device__ __forceinline__ void load_gu_row(uint64_t slice, uint32_t proj, int k, unsigned n, int nch, int c,
                                            LaneRaw& r) {
  if (GU == TQ4_KM) load_km(reinterpret_cast<const uint8_t*>(slice), k, n, c, r);
  else load_raw<GU>(reinterpret_cast<const uint8_t*>(slice) + (k ? proj : 0) + (size_t)n * (proj / kNeurons), nch, c, r);
}

// Scale factors of the raw row for the fp32 path; false on a bad scale.
template <int type>
__device__ __forceinline__ bool raw_scales(const LaneRaw& r, int c, float s[2], float m[2]) {
  if (type == TQ4_K) {
    float d = half_to_float(r.h.x & 0xffff), dm = half_to_float(r.h.x >> 16);
    uint32_t g0 = 2 * (c & 3), sc0, mi0, sc1, mi1;
    q4k_scale_min(r.h.y, r.h.z, r.h.w, g0, sc0, mi0);
    q4k_scale_min(r.h.y, r.h.z, r.h.w, g0 + 1, sc1, mi1);
    s[0] = d * (float)sc0;
    s[1] = d * (float)sc1;
    m[0] = dm * (float)mi0;
    m[1] = dm * (float)mi1;
    return !half_bad(r.h.x) && !half_bad(r.h.x >> 16);
  } else if (type == TMXFP4) {
    s[0] = e8m0(r.h.x & 0xff);
    s[1] = e8m0((r.h.x >> 8) & 0xff);
    m[0] = m[1] = 0.f;
    return !mx_blocks_bad(r.h.x & 0xff, r.q[0], (r.h.x >> 8) & 0xff, r.q[1]);
  } else {  // Q8_0, Q4_0: two fp16 scales
    s[0] = half_to_float(r.h.x & 0xffff);
    s[1] = half_to_float(r.h.x >> 16);
    m[0] = m[1] = 0.f;
    return !half_bad(r.h.x) && !half_bad(r.h.x >> 16);
  }
}

// Exact reference decode of the raw row (src/native.c:13-31, src/q4.c:29-31).
template <int type>
__device__ __forceinline__ bool decode_raw(const LaneRaw& r, int c, float* w) {
  float s[2], m[2];
  bool ok = raw_scales<type>(r, c, s, m);
  if (type == TQ4_K) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t v = word(r.q[i >> 2], i & 3);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t byte = v >> (8 * b);
        w[4 * i + b] = fmaf(s[0], (float)(byte & 15u), -m[0]);
        w[32 + 4 * i + b] = fmaf(s[1], (float)((byte >> 4) & 15u), -m[1]);
      }
    }
  } else if (type == TQ8_0) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v = word(r.q[p], i);
#pragma unroll
        for (int b = 0; b < 4; ++b) w[16 * p + 4 * i + b] = (p < 2 ? s[0] : s[1]) * (float)(int8_t)(v >> (8 * b));
      }
  } else if (type == TMXFP4) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v = word(r.q[p], i);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float2 e = fp4_pair(v, s[p], b);
          w[32 * p + 4 * i + b] = e.x + 0.0f;   // -0 -> +0 as the reference table
          w[32 * p + 16 + 4 * i + b] = e.y + 0.0f;
        }
      }
  } else {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v = word(r.q[p], i);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          uint32_t byte = v >> (8 * b);
          w[32 * p + 4 * i + b] = (float)((int)(byte & 15u) - 8) * s[p];
          w[32 * p + 16 + 4 * i + b] = (float)((int)((byte >> 4) & 15u) - 8) * s[p];
        }
      }
  }
  return ok;
}

__device__ bool decode_lane(uint8_t type, const uint8_t* row, int nch, int c, float* w) {
  LaneRaw r;
  switch (type) {
    case TQ4_K: load_raw<TQ4_K>(row, nch, c, r); return decode_raw<TQ4_K>(r, c, w);
    case TQ8_0: load_raw<TQ8_0>(row, nch, c, r); return decode_raw<TQ8_0>(r, c, w);
    case TMXFP4: load_raw<TMXFP4>(row, nch, c, r); return decode_raw<TMXFP4>(r, c, w);
    default: load_raw<TQ4_0>(row, nch, c, r); return decode_raw<TQ4_0>(r, c, w);
  }
}

// fp32 partial of one lane for one token. x points at the lane's 64
// activations; X0/X1 are the sums of x[0..31] and x[32..63]. The Q4_K and
// Q4_0 forms factor the scale and min out of the 32-column groups:
// sum_j (D*q_j - M)*x_j = D*sum_j q_j*x_j - M*sum_j x_j.
template <int type>
__device__ __forceinline__ float lane_dot_f32(const LaneRaw& r, const float* sc, const float* mn, const float4* x,
                                              float X0, float X1) {
  float s0 = 0.f, s1 = 0.f;
  if (type == TQ4_K) {
    // Byte i of the 32-byte chunk: column i (low nibble), 32+i (high). Eight
    // independent chains (one per byte position and nibble) so that the
    // FMAs of a wave do not wait on each other. Nibbles two per conversion
    // as q * 2^-9 (nib_pair); the sums are those of q times 2^-9 exactly.
    float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = word(r.q[i >> 2], i & 3);
      const uint32_t lo = nib_lo(v), hi = nib_hi(v);
      const float4 xa = x[i], xb = x[8 + i];
      const float2 l01 = nib_pair<false>(lo), l23 = nib_pair<true>(lo);
      const float2 h01 = nib_pair<false>(hi), h23 = nib_pair<true>(hi);
      a[0] = fmaf(l01.x, xa.x, a[0]);
      a[1] = fmaf(l01.y, xa.y, a[1]);
      a[2] = fmaf(l23.x, xa.z, a[2]);
      a[3] = fmaf(l23.y, xa.w, a[3]);
      b[0] = fmaf(h01.x, xb.x, b[0]);
      b[1] = fmaf(h01.y, xb.y, b[1]);
      b[2] = fmaf(h23.x, xb.z, b[2]);
      b[3] = fmaf(h23.y, xb.w, b[3]);
    }
    s0 = ((a[0] + a[1]) + (a[2] + a[3])) * kFp8Nibble;
    s1 = ((b[0] + b[1]) + (b[2] + b[3])) * kFp8Nibble;
    return (sc[0] * s0 - mn[0] * X0) + (sc[1] * s1 - mn[1] * X1);
  }
  if (type == TQ4_0) {
    // Per 32-column block p, byte i: column i (low nibble), 16+i (high).
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = word(r.q[p], i);
        const uint32_t lo = nib_lo(v), hi = nib_hi(v);
        const float4 a = x[8 * p + i], b = x[8 * p + 4 + i];
        const float2 l01 = nib_pair<false>(lo), l23 = nib_pair<true>(lo);
        const float2 h01 = nib_pair<false>(hi), h23 = nib_pair<true>(hi);
        s = fmaf(l01.x, a.x, s);
        s = fmaf(l01.y, a.y, s);
        s = fmaf(l23.x, a.z, s);
        s = fmaf(l23.y, a.w, s);
        s = fmaf(h01.x, b.x, s);
        s = fmaf(h01.y, b.y, s);
        s = fmaf(h23.x, b.z, s);
        s = fmaf(h23.y, b.w, s);
      }
      s *= kFp8Nibble;   // the sum of q * x (nib_pair's 2^-9 undone exactly)
      if (p) s1 = s; else s0 = s;
    }
    return sc[0] * (s0 - 8.f * X0) + sc[1] * (s1 - 8.f * X1);
  }
  if (type == TQ8_0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = word(r.q[p], i);
        const float4 a = x[4 * p + i];
        s = fmaf((float)(int8_t)v, a.x, s);
        s = fmaf((float)(int8_t)(v >> 8), a.y, s);
        s = fmaf((float)(int8_t)(v >> 16), a.z, s);
        s = fmaf((float)(int8_t)(v >> 24), a.w, s);
      }
      if (p < 2) s0 += s; else s1 += s;
    }
    return sc[0] * s0 + sc[1] * s1;
  }
  // MXFP4: per 32-column block p, byte i holds element i (low) and 16+i.
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = word(r.q[p], i);
      const float4 a = x[8 * p + i], b = x[8 * p + 4 + i];
      float2 e0 = fp4_pair(v, 1.0f, 0), e1 = fp4_pair(v, 1.0f, 1), e2 = fp4_pair(v, 1.0f, 2), e3 = fp4_pair(v, 1.0f, 3);
      s = fmaf(e0.x, a.x, s);
      s = fmaf(e1.x, a.y, s);
      s = fmaf(e2.x, a.z, s);
      s = fmaf(e3.x, a.w, s);
      s = fmaf(e0.y, b.x, s);
      s = fmaf(e1.y, b.y, s);
      s = fmaf(e2.y, b.z, s);
      s = fmaf(e3.y, b.w, s);
    }
    if (p) s1 = s; else s0 = s;
  }
  return sc[0] * s0 + sc[1] * s1;
}

// ------------------------------------------------------------ phase A
//
// Task (pair p, neuron group ng of kTaskNeurons): 4 wavefronts, each owning
// kWaveNeurons neurons (a gate row and an up row each). Lane c of a wave owns
// activation columns 64c..64c+63 of every row it streams; a DPP tree reduces
// each row to a wave-uniform value. Each wave publishes its own h values and
// releases the pair counter once, so a pair is complete at kDoneTarget.

constexpr int kTaskNeurons = 8;
constexpr int kWaveNeurons = kTaskNeurons / kWaves;
constexpr uint32_t kDoneTarget = (kNeurons / kTaskNeurons) * kWaves;

__device__ __forceinline__ float silu_mul(float a, float u, uint32_t& bad) {
  if (!isfinite(a) || !isfinite(u)) {
    bad |= kErrRange;
    return 0.f;
  }
  // Stable sigmoid in double, as backends/ref.c:82-83.
  double ad = a;
  double sig = ad >= 0 ? 1.0 / (1.0 + exp(-ad)) : exp(ad) / (1.0 + exp(ad));
  double hv = ad * sig * (double)u;
  if (!isfinite(hv) || fabs(hv) > (double)FLT_MAX) {
    bad |= kErrRange;
    return 0.f;
  }
  return (float)hv;
}

__device__ __forceinline__ float narrow_dot(double s) {
  return (!isfinite(s) || fabs(s) > (double)FLT_MAX) ? INFINITY : (float)s;
}

__device__ __forceinline__ void publish_h(const Scratch& S, size_t index, float h) { put(S.hbuf + index, h); }

// The wave's h stores are complete (drained) before its pair counter moves.
__device__ __forceinline__ void release_pair(const Scratch& S, unsigned p) {
  drain_stores();
  if ((threadIdx.x & 63) == 0) bump(S.done + (size_t)S.parity * kMaxPairs + p);
}

// Single token: the lane's 64 activations live in registers, every row load
// of the wave is issued before any arithmetic, no LDS and no barrier.
template <int MODE, int GU>
__device__ __forceinline__ uint32_t phase_a_single(const PlanHeader& H, const Scratch& S, unsigned p, unsigned n0,
                                                   uint64_t slice, uint32_t proj, const float* xg) {
  const unsigned nch = H.hidden / 64;
  const int lane = threadIdx.x & 63;
  const bool active = lane < (int)nch;
  const int c = active ? lane : 0;
  LaneRaw raw[2 * kWaveNeurons];
#pragma unroll
  for (int k = 0; k < kWaveNeurons; ++k)
#pragma unroll
    for (int r = 0; r < 2; ++r)
      load_gu_row<GU>(slice, proj, r, n0 + k, nch, c, raw[2 * k + r]);
  float4 x[16];
  {
    const float4* xs = reinterpret_cast<const float4*>(xg + 64 * c);
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = xs[i];
  }
  if (MODE == MODE_Q8) q8_regs64(x);  // the lane chunk is one 64-group
  float X0 = 0.f, X1 = 0.f;
  if (MODE == MODE_F32 && (kAs<GU> == TQ4_K || GU == TQ4_0)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      X0 += (x[i].x + x[i].y) + (x[i].z + x[i].w);
      X1 += (x[8 + i].x + x[8 + i].y) + (x[8 + i].z + x[8 + i].w);
    }
  }
  uint32_t bad = 0;
#pragma unroll
  for (int k = 0; k < kWaveNeurons; ++k) {
    float au[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const LaneRaw& rr = raw[2 * k + r];
      if (MODE == MODE_F32) {
        float sc[2], mn[2];
        bool ok = raw_scales<kAs<GU>>(rr, c, sc, mn);
        if (active && !ok) bad |= kErrScale;
        float part = lane_dot_f32<kAs<GU>>(rr, sc, mn, x, X0, X1);
        au[r] = wave_total(active ? part : 0.f);
      } else {
        float w[64];
        bool ok = decode_raw<kAs<GU>>(rr, c, w);
        if (active && !ok) bad |= kErrScale;
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          acc = fma((double)w[4 * j], (double)x[j].x, acc);
          acc = fma((double)w[4 * j + 1], (double)x[j].y, acc);
          acc = fma((double)w[4 * j + 2], (double)x[j].z, acc);
          acc = fma((double)w[4 * j + 3], (double)x[j].w, acc);
        }
        au[r] = narrow_dot(wave_total(active ? acc : 0.0));
      }
    }
    float h = silu_mul(au[0], au[1], bad);
    if (lane == 0) publish_h(S, (size_t)p * kMaxBurst * kNeurons + n0 + k, h);
  }
  return bad;
}

// Bursts: activations of up to BT tokens staged in LDS per tile; each row's
// loaded bytes are reused for every token of the tile.
template <int MODE, int BT, int GU>
__device__ __forceinline__ uint32_t phase_a_tile(const PlanHeader& H, const Scratch& S, unsigned p, unsigned n0,
                                                 uint64_t slice, uint32_t proj, uint32_t tmask, unsigned t0,
                                                 unsigned tc, const float* lds) {
  const unsigned hidden = H.hidden, nch = hidden / 64;
  const int lane = threadIdx.x & 63;
  const bool active = lane < (int)nch;
  const int c = active ? lane : 0;
  uint32_t bad = 0;
  float X0[BT], X1[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) {
    X0[t] = X1[t] = 0.f;
    if (MODE == MODE_F32 && (kAs<GU> == TQ4_K || GU == TQ4_0) && t < (int)tc) {
      const float4* x = reinterpret_cast<const float4*>(lds + t * hidden + 64 * c);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float4 a = x[i], b = x[8 + i];
        X0[t] += (a.x + a.y) + (a.z + a.w);
        X1[t] += (b.x + b.y) + (b.z + b.w);
      }
    }
  }
  LaneRaw raw[2 * kWaveNeurons];
#pragma unroll
  for (int k = 0; k < kWaveNeurons; ++k)
#pragma unroll
    for (int r = 0; r < 2; ++r)
      load_gu_row<GU>(slice, proj, r, n0 + k, nch, c, raw[2 * k + r]);
#pragma unroll
  for (int k = 0; k < kWaveNeurons; ++k) {
    float au[2][BT];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const LaneRaw& rr = raw[2 * k + r];
      if (MODE == MODE_F32) {
        float sc[2], mn[2];
        bool ok = raw_scales<kAs<GU>>(rr, c, sc, mn);
        if (active && !ok) bad |= kErrScale;
#pragma unroll
        for (int t = 0; t < BT; ++t) {
          float part = 0.f;
          if (active && t < (int)tc)
            part = lane_dot_f32<kAs<GU>>(rr, sc, mn, reinterpret_cast<const float4*>(lds + t * hidden + 64 * c), X0[t], X1[t]);
          au[r][t] = wave_total(part);
        }
      } else {
        float w[64];
        bool ok = decode_raw<kAs<GU>>(rr, c, w);
        if (active && !ok) bad |= kErrScale;
#pragma unroll
        for (int t = 0; t < BT; ++t) {
          double acc = 0.0;
          if (active && t < (int)tc) {
            const float* x = lds + t * hidden + 64 * c;
#pragma unroll
            for (int j = 0; j < 64; ++j) acc = fma((double)w[j], (double)x[j], acc);
          }
          au[r][t] = narrow_dot(wave_total(acc));
        }
      }
    }
#pragma unroll
    for (int t = 0; t < BT; ++t) {
      if (t >= (int)tc || !((tmask >> (t0 + t)) & 1u)) continue;
      float h = silu_mul(au[0][t], au[1][t], bad);
      if (lane == 0) publish_h(S, ((size_t)p * kMaxBurst + t0 + t) * kNeurons + n0 + k, h);
    }
  }
  return bad;
}

template <int MODE, int BT>
__device__ void phase_a(const PlanHeader& H, const uint8_t* plan, const Scratch& S, uint32_t* status,
                        unsigned task, float* lds) {
  constexpr unsigned per_pair = kNeurons / kTaskNeurons;
  const unsigned p = task / per_pair, ng = task % per_pair;
  const PairDesc* P = reinterpret_cast<const PairDesc*>(plan + H.pairs_off) + p;
  const uint64_t slice = P->slice;
  const uint32_t proj = P->proj;
  const uint8_t gu = P->gu;
  const uint32_t tmask = P->tmask;
  const unsigned hidden = H.hidden, nch = hidden / 64, T = H.burst;
  const unsigned n0 = ng * kTaskNeurons + (threadIdx.x >> 6) * kWaveNeurons;
  const float* xg = reinterpret_cast<const float*>(plan + H.x_off);
  uint32_t bad = 0;
  if (BT == 1) {
    switch (gu) {
      case TQ4_K: bad = phase_a_single<MODE, TQ4_K>(H, S, p, n0, slice, proj, xg); break;
      case TQ4_KM: bad = phase_a_single<MODE, TQ4_KM>(H, S, p, n0, slice, proj, xg); break;
      case TQ8_0: bad = phase_a_single<MODE, TQ8_0>(H, S, p, n0, slice, proj, xg); break;
      case TMXFP4: bad = phase_a_single<MODE, TMXFP4>(H, S, p, n0, slice, proj, xg); break;
      default: bad = phase_a_single<MODE, TQ4_0>(H, S, p, n0, slice, proj, xg); break;
    }
  } else {
    for (unsigned t0 = 0; t0 < T; t0 += BT) {
      const unsigned tc = min((unsigned)BT, T - t0);
      if (t0) __syncthreads();
      {
        const float4* src = reinterpret_cast<const float4*>(xg + (size_t)t0 * hidden);
        float4* dst = reinterpret_cast<float4*>(lds);
        for (unsigned i = threadIdx.x; i < tc * hidden / 4; i += kThreads) dst[i] = src[i];
      }
      __syncthreads();
      if (MODE == MODE_Q8) {
        for (unsigned g = threadIdx.x; g < tc * nch; g += kThreads) q8_group(lds + 64 * g, 64);
        __syncthreads();
      }
      switch (gu) {
        case TQ4_K: bad |= phase_a_tile<MODE, BT, TQ4_K>(H, S, p, n0, slice, proj, tmask, t0, tc, lds); break;
        case TQ4_KM: bad |= phase_a_tile<MODE, BT, TQ4_KM>(H, S, p, n0, slice, proj, tmask, t0, tc, lds); break;
        case TQ8_0: bad |= phase_a_tile<MODE, BT, TQ8_0>(H, S, p, n0, slice, proj, tmask, t0, tc, lds); break;
        case TMXFP4: bad |= phase_a_tile<MODE, BT, TMXFP4>(H, S, p, n0, slice, proj, tmask, t0, tc, lds); break;
        default: bad |= phase_a_tile<MODE, BT, TQ4_0>(H, S, p, n0, slice, proj, tmask, t0, tc, lds); break;
      }
    }
  }
  if (bad) flag(status, bad);
  release_pair(S, p);
}

// ------------------------------------------------------------ phase B
//
// Down matrices, re-tiled:
//  MXFP4 [H x 32]: [H][16 B] codes (byte i: neuron i low, 16+i high), [H] E8M0.
//  Q8_0  [H x 32]: [2 parts][H][16 B] int8, then [H][fp16].
//  Q4_0  [H x 32]: [H][16 B] nibbles (byte i: neuron i low, 16+i high), [H][fp16].
//  Q4_K transposed [32 x H]: per 256-column super-block, [4][64 lanes][16 B]
//         nibbles, lane l holding columns 4l..4l+3 of neurons 8k..8k+7 (dword
//         w: neurons 8k+2w, 8k+2w+1; nibble j: neuron +j/4, column +j%4),
//         then the 32 neurons' 16-byte super-block headers.

__device__ __forceinline__ void hdr_dm(const uint4& h, uint32_t g, float& D, float& M, bool& ok) {
  ok = !half_bad(h.x) && !half_bad(h.x >> 16);
  uint32_t sc, mi;
  q4k_scale_min(h.y, h.z, h.w, g, sc, mi);
  D = half_to_float(h.x & 0xffff) * (float)sc;
  M = half_to_float(h.x >> 16) * (float)mi;
}

// Decode one [H x 32] down row (neurons 0..31 of output d) exactly.
__device__ bool decode_down_row(uint8_t dn, const uint8_t* down, unsigned hidden, unsigned d, float* w) {
  bool ok = true;
  if (dn == TMXFP4) {
    uint4 q = ld16(down + 16 * (size_t)d);
    uint32_t e = down[16 * (size_t)hidden + d];
    ok = !mx_block_bad(e, q);
    float sc = e8m0(e);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t v = word(q, i);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        float2 f = fp4_pair(v, sc, b);
        w[4 * i + b] = f.x + 0.0f;
        w[16 + 4 * i + b] = f.y + 0.0f;
      }
    }
  } else if (dn == TQ8_0) {
    uint32_t s = reinterpret_cast<const uint16_t*>(down + 32 * (size_t)hidden)[d];
    ok = !half_bad(s);
    float sc = half_to_float(s);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      uint4 q = ld16(down + 16 * (size_t)hidden * p + 16 * (size_t)d);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v = word(q, i);
#pragma unroll
        for (int b = 0; b < 4; ++b) w[16 * p + 4 * i + b] = sc * (float)(int8_t)(v >> (8 * b));
      }
    }
  } else {  // Q4_0
    uint32_t s = reinterpret_cast<const uint16_t*>(down + 16 * (size_t)hidden)[d];
    ok = !half_bad(s);
    float sc = half_to_float(s);
    uint4 q = ld16(down + 16 * (size_t)d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t v = word(q, i);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t byte = v >> (8 * b);
        w[4 * i + b] = (float)((int)(byte & 15u) - 8) * sc;
        w[16 + 4 * i + b] = (float)((int)((byte >> 4) & 15u) - 8) * sc;
      }
    }
  }
  return ok;
}

// Decode the 4 columns x 32 neurons of lane l in super-block sb of a
// transposed Q4_K down matrix: w[n*4 + c] (exact reference decode).
__device__ bool decode_down_q4kt(const uint8_t* down, unsigned sb, int l, float* w) {
  const uint8_t* base = down + 4608 * (size_t)sb;
  bool ok = true;
  const uint32_t g = (uint32_t)l >> 3;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint4 q = ld16(base + 1024 * k + 16 * l);
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      uint32_t v = word(q, wd);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        int n = 8 * k + 2 * wd + s;
        uint4 h = ld16(base + 4096 + 16 * n);
        float D, M;
        bool hok;
        hdr_dm(h, g, D, M, hok);
        ok &= hok;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) w[4 * n + cc] = fmaf(D, (float)((v >> (4 * (4 * s + cc))) & 15u), -M);
      }
    }
  }
  return ok;
}

// Wait (bounded) until every pair of the group has all 32 h values, then
// stage them in LDS (Q8 mode: quantized per slice, backends/ref.c:85).
// Called by the whole workgroup after it issued its weight loads.
template <int MODE>
__device__ __forceinline__ uint32_t stage_h(const PlanHeader& H, const Scratch& S, const GroupDesc& G, float* hs) {
  const unsigned T = H.burst, count = G.count;
  uint32_t bad = 0;
  if (threadIdx.x == 0) {
    for (unsigned j = 0; j < count; ++j) {
      const uint32_t* ctr = S.done + (size_t)S.parity * kMaxPairs + G.first + j;
      uint32_t spins = 0;
      while (get(ctr) < kDoneTarget) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kSpinLimit) {
          bad |= kErrTimeout;
          break;
        }
      }
    }
  }
  __syncthreads();
  for (unsigned i = threadIdx.x; i < count * T * kNeurons; i += kThreads) {
    unsigned j = i / (T * kNeurons), r = i % (T * kNeurons);
    hs[i] = get(S.hbuf + ((size_t)(G.first + j) * kMaxBurst) * kNeurons + r);
  }
  __syncthreads();
  if (MODE == MODE_Q8) {
    for (unsigned i = threadIdx.x; i < count * T; i += kThreads) q8_group(hs + i * kNeurons, kNeurons);
    __syncthreads();
  }
  return bad;
}

template <int DN>
constexpr int group_max() { return DN == TQ8_0 ? 6 : DN == TQ4_KT ? 8 : 12; }

// [H x 32] down formats: thread = output row d of the 256-row range; every
// pair of the group is prefetched before the dependency wait.
template <int MODE, int TB, int DN>
__device__ __forceinline__ uint32_t phase_b_rows(const PlanHeader& H, const Scratch& S, const GroupDesc& G,
                                                 const PairDesc* pairs, unsigned gi, unsigned cr, float* hs) {
  constexpr int MAXG = group_max<DN>();
  const unsigned hidden = H.hidden, T = H.burst, count = G.count;
  const unsigned d = cr * kCols + threadIdx.x;
  uint4 q0[MAXG], q1[MAXG];
  uint32_t sw[MAXG];
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    q0[j] = q1[j] = make_uint4(0, 0, 0, 0);
    sw[j] = 0;
    if (j >= (int)count) continue;
    const PairDesc* P = pairs + G.first + j;
    const uint8_t* down = reinterpret_cast<const uint8_t*>(P->slice) + 2 * (size_t)P->proj;
    q0[j] = ld16(down + 16 * (size_t)d);
    if (DN == TQ8_0) {
      q1[j] = ld16(down + 16 * (size_t)hidden + 16 * (size_t)d);
      sw[j] = gld<uint16_t>(down + 32 * (size_t)hidden + 2 * (size_t)d);
    } else if (DN == TMXFP4) {
      sw[j] = gld<uint8_t>(down + 16 * (size_t)hidden + d);
    } else {
      sw[j] = gld<uint16_t>(down + 16 * (size_t)hidden + 2 * (size_t)d);
    }
  }
  uint32_t bad = stage_h<MODE>(H, S, G, hs);
  double y[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) y[t] = 0.0;
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    if (j >= (int)count) continue;
    const PairDesc* P = pairs + G.first + j;
    const uint32_t tmask = P->tmask;
    if (MODE == MODE_F32) {
      float sc;
      if (DN == TMXFP4) {
        if (mx_block_bad(sw[j], q0[j])) bad |= kErrScale;
        sc = e8m0(sw[j]);
      } else {
        if (half_bad(sw[j])) bad |= kErrScale;
        sc = half_to_float(sw[j]);
      }
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (t >= (int)T || !((tmask >> t) & 1u)) continue;
        const float4* h4 = reinterpret_cast<const float4*>(hs + (j * T + t) * kNeurons);
        float sum = 0.f;
        if (DN == TQ8_0) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t v = word(i < 4 ? q0[j] : q1[j], i & 3);
            const float4 h = h4[i];
            sum = fmaf((float)(int8_t)v, h.x, sum);
            sum = fmaf((float)(int8_t)(v >> 8), h.y, sum);
            sum = fmaf((float)(int8_t)(v >> 16), h.z, sum);
            sum = fmaf((float)(int8_t)(v >> 24), h.w, sum);
          }
        } else {
          // Byte i: neuron i (low nibble), neuron 16+i (high nibble).
          float hsum = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t v = word(q0[j], i);
            const float4 a = h4[i], b = h4[4 + i];
            if (DN == TMXFP4) {
              float2 e0 = fp4_pair(v, 1.0f, 0), e1 = fp4_pair(v, 1.0f, 1), e2 = fp4_pair(v, 1.0f, 2),
                     e3 = fp4_pair(v, 1.0f, 3);
              sum = fmaf(e0.x, a.x, sum);
              sum = fmaf(e1.x, a.y, sum);
              sum = fmaf(e2.x, a.z, sum);
              sum = fmaf(e3.x, a.w, sum);
              sum = fmaf(e0.y, b.x, sum);
              sum = fmaf(e1.y, b.y, sum);
              sum = fmaf(e2.y, b.z, sum);
              sum = fmaf(e3.y, b.w, sum);
            } else {
              sum = fmaf((float)(v & 15u), a.x, sum);
              sum = fmaf((float)((v >> 8) & 15u), a.y, sum);
              sum = fmaf((float)((v >> 16) & 15u), a.z, sum);
              sum = fmaf((float)((v >> 24) & 15u), a.w, sum);
              sum = fmaf((float)((v >> 4) & 15u), b.x, sum);
              sum = fmaf((float)((v >> 12) & 15u), b.y, sum);
              sum = fmaf((float)((v >> 20) & 15u), b.z, sum);
              sum = fmaf((float)(v >> 28), b.w, sum);
              hsum += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
            }
          }
          if (DN == TQ4_0) sum -= 8.f * hsum;
        }
        y[t] += (double)P->gate[t] * ((double)sc * (double)sum);
      }
    } else {
      // Exact decode of the row (decode_down_row semantics) from registers.
      float w[32];
      if (DN == TMXFP4) {
        if (mx_block_bad(sw[j], q0[j])) bad |= kErrScale;
        const float sc = e8m0(sw[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t v = word(q0[j], i);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const float2 f = fp4_pair(v, sc, b);
            w[4 * i + b] = f.x;
            w[16 + 4 * i + b] = f.y;
          }
        }
      } else if (DN == TQ8_0) {
        if (half_bad(sw[j])) bad |= kErrScale;
        const float sc = half_to_float(sw[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t v = word(i < 4 ? q0[j] : q1[j], i & 3);
#pragma unroll
          for (int b = 0; b < 4; ++b) w[4 * i + b] = sc * (float)(int8_t)(v >> (8 * b));
        }
      } else {
        if (half_bad(sw[j])) bad |= kErrScale;
        const float sc = half_to_float(sw[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t v = word(q0[j], i);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            w[4 * i + b] = (float)((int)((v >> (8 * b)) & 15u) - 8) * sc;
            w[16 + 4 * i + b] = (float)((int)((v >> (8 * b + 4)) & 15u) - 8) * sc;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (t >= (int)T || !((tmask >> t) & 1u)) continue;
        const float* h = hs + (j * T + t) * kNeurons;
        double sum = 0.0;
#pragma unroll
        for (int n = 0; n < 32; ++n) sum = fma((double)w[n], (double)h[n], sum);
        y[t] += (double)P->gate[t] * sum;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TB; ++t)
    if (t < (int)T) put(S.partial + ((size_t)gi * T + t) * hidden + d, y[t]);
  return bad;
}

// Transposed Q4_K down: lane l covers columns 4l..4l+3 of super-block cr
// (group g = l/8); wave w takes pairs w and w+4. The 8 lanes of a group
// decode the scales of 4 neurons each and share them through a per-wave LDS
// table (row stride 36 floats keeps the 8 groups on distinct banks).
constexpr int kTabStride = 36;

template <int MODE, int TB>
__device__ __forceinline__ uint32_t phase_b_q4kt(const PlanHeader& H, const Scratch& S, const GroupDesc& G,
                                                 const PairDesc* pairs, unsigned gi, unsigned cr, float* hs,
                                                 float* wtab, double* red) {
  const unsigned hidden = H.hidden, T = H.burst, count = G.count;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t g = (uint32_t)lane >> 3, nb = 4 * (lane & 7);
  uint4 q[2][4], hd[2][4];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const unsigned j = wave + kWaves * jj;
#pragma unroll
    for (int k = 0; k < 4; ++k) q[jj][k] = hd[jj][k] = make_uint4(0, 0, 0, 0);
    if (j >= count) continue;
    const PairDesc* P = pairs + G.first + j;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(P->slice) + 2 * (size_t)P->proj + 4608 * (size_t)cr;
#pragma unroll
    for (int k = 0; k < 4; ++k) q[jj][k] = ld16(base + 1024 * k + 16 * lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) hd[jj][i] = ld16(base + 4096 + 16 * (nb + i));
  }
  uint32_t bad = stage_h<MODE>(H, S, G, hs);
  const unsigned wstride = 2 * 8 * kTabStride + T * 8 * kTabStride;
  float* tD = wtab + wave * wstride;
  float* tM = tD + 8 * kTabStride;
  float* cD = tM + 8 * kTabStride;
  double y[TB][4];
#pragma unroll
  for (int t = 0; t < TB; ++t)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) y[t][cc] = 0.0;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const unsigned j = wave + kWaves * jj;
    if (j >= count) continue;
    const PairDesc* P = pairs + G.first + j;
    const uint32_t tmask = P->tmask;
    float D[4], M[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bool ok;
      hdr_dm(hd[jj][i], g, D[i], M[i], ok);
      if (!ok) bad |= kErrScale;
    }
    float B[TB];
    if (MODE == MODE_F32) {
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        B[t] = 0.f;
        if (t >= (int)T) continue;
        const float* h = hs + (j * T + t) * kNeurons;
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cD[t * 8 * kTabStride + g * kTabStride + nb + i] = D[i] * h[nb + i];
          part = fmaf(M[i], h[nb + i], part);
        }
        B[t] = oct_sum(part);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tD[g * kTabStride + nb + i] = D[i];
        tM[g * kTabStride + nb + i] = M[i];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (t >= (int)T || !((tmask >> t) & 1u)) continue;
      const double gate = (double)P->gate[t];
      if (MODE == MODE_F32) {
        const float4* cd = reinterpret_cast<const float4*>(cD + t * 8 * kTabStride + g * kTabStride);
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 c0 = cd[2 * k], c1 = cd[2 * k + 1];  // neurons 8k..8k+7
          const float coef[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
          for (int wd = 0; wd < 4; ++wd) {
            // Nibble j of the dword: neuron 2wd + j/4, column j%4. Low nibbles
            // of bytes 0..3 are j = 0,2,4,6; high nibbles j = 1,3,5,7.
            const uint32_t v = word(q[jj][k], wd);
            const uint32_t lo = nib_lo(v), hi = nib_hi(v);
            const float ca = coef[2 * wd], cb = coef[2 * wd + 1];
            s4[0] = fmaf(ub(lo, 0), ca, s4[0]);
            s4[1] = fmaf(ub(hi, 0), ca, s4[1]);
            s4[2] = fmaf(ub(lo, 1), ca, s4[2]);
            s4[3] = fmaf(ub(hi, 1), ca, s4[3]);
            s4[0] = fmaf(ub(lo, 2), cb, s4[0]);
            s4[1] = fmaf(ub(hi, 2), cb, s4[1]);
            s4[2] = fmaf(ub(lo, 3), cb, s4[2]);
            s4[3] = fmaf(ub(hi, 3), cb, s4[3]);
          }
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) y[t][cc] += gate * (double)(s4[cc] - B[t]);
      } else {
        const float* h = hs + (j * T + t) * kNeurons;
        double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int wd = 0; wd < 4; ++wd) {
            const uint32_t v = word(q[jj][k], wd);
#pragma unroll
            for (int sN = 0; sN < 2; ++sN) {
              const int n = 8 * k + 2 * wd + sN;
              const float Dn = tD[g * kTabStride + n], Mn = tM[g * kTabStride + n];
              const double hn = (double)h[n];
#pragma unroll
              for (int cc = 0; cc < 4; ++cc)
                s4[cc] = fma((double)fmaf(Dn, (float)((v >> (4 * (4 * sN + cc))) & 15u), -Mn), hn, s4[cc]);
            }
          }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) y[t][cc] += gate * s4[cc];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    if (t >= (int)T) continue;
    __syncthreads();
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) red[wave * kCols + 4 * lane + cc] = y[t][cc];
    __syncthreads();
    const int tid = threadIdx.x;
    const double v = ((red[tid] + red[kCols + tid]) + red[2 * kCols + tid]) + red[3 * kCols + tid];
    put(S.partial + ((size_t)gi * T + t) * hidden + cr * kCols + tid, v);
  }
  return bad;
}

template <int MODE, int TB>
__device__ void phase_b(const PlanHeader& H, const uint8_t* plan, const Scratch& S, uint32_t* status,
                        unsigned task, float* lds) {
  const unsigned gi = task / H.nranges, cr = task % H.nranges;
  const GroupDesc G = reinterpret_cast<const GroupDesc*>(plan + H.groups_off)[gi];
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + H.pairs_off);
  const unsigned hidden = H.hidden, T = H.burst;
  const int tid = threadIdx.x;
  // LDS: hs[gmax][T][32] | 4 per-wave scale tables | wave reduction.
  float* hs = lds;
  const unsigned wstride = 2 * 8 * kTabStride + T * 8 * kTabStride;
  float* wtab = hs + H.gmax * T * kNeurons;
  double* red = reinterpret_cast<double*>(wtab + kWaves * wstride);
  uint32_t bad;
  switch (G.dn) {
    case TQ4_KT: bad = phase_b_q4kt<MODE, TB>(H, S, G, pairs, gi, cr, hs, wtab, red); break;
    case TMXFP4: bad = phase_b_rows<MODE, TB, TMXFP4>(H, S, G, pairs, gi, cr, hs); break;
    case TQ8_0: bad = phase_b_rows<MODE, TB, TQ8_0>(H, S, G, pairs, gi, cr, hs); break;
    default: bad = phase_b_rows<MODE, TB, TQ4_0>(H, S, G, pairs, gi, cr, hs); break;
  }
  if (bad) flag(status, bad);

  // The last-arriving group of this output range reduces it, in group order.
  // Every thread drains its partial stores before the ticket is taken.
  __shared__ uint32_t ticket;
  drain_stores();
  __syncthreads();
  if (tid == 0) ticket = bump(S.fin + (size_t)S.parity * kMaxRanges + cr);
  __syncthreads();
  if (ticket != H.ngroups - 1) return;
  float* yout = reinterpret_cast<float*>(status + 4);
  const unsigned col = cr * kCols + tid;
  for (unsigned t = 0; t < T; ++t) {
    double v = 0.0;
    for (unsigned g2 = 0; g2 < H.ngroups; ++g2) v += get(S.partial + ((size_t)g2 * T + t) * hidden + col);
    float f = 0.f;
    if (!isfinite(v) || fabs(v) > (double)FLT_MAX) flag(status, kErrRange);
    else f = (float)v;
    yout[(size_t)t * hidden + col] = f;
  }
}

// TILE = 1 for single-token requests, 8 for bursts (phase A in tiles of 4).
// Clear the other parity's counters and status for the next launch (whichever
// kernel it runs). Called by workgroup 0.
__device__ __forceinline__ void clear_other_parity(const Scratch& S) {
  const uint32_t other = S.parity ^ 1u;
  for (unsigned i = threadIdx.x; i < kMaxPairs; i += blockDim.x) S.done[(size_t)other * kMaxPairs + i] = 0;
  if (threadIdx.x < kMaxRanges) S.fin[(size_t)other * kMaxRanges + threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    S.out[(size_t)other * S.out_words] = 0;
    S.bar[other] = 0;
  }
}

template <int MODE, int TILE>
__global__ __launch_bounds__(kThreads) void layer_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  extern __shared__ __align__(16) float lds[];
  const PlanHeader H = *reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = S.out + (size_t)S.parity * S.out_words;
  if (blockIdx.x == 0) clear_other_parity(S);
  const unsigned b = blockIdx.x;
  if (b < H.ntA) phase_a<MODE, TILE == 1 ? 1 : 4>(H, plan, S, status, b, lds);
  else phase_b<MODE, TILE>(H, plan, S, status, b - H.ntA, lds);
}

// ------------------------------------------------------------ decode kernel
//
// F32 mode, every pair routed Q4_K (TQ4_KM tiles) with the transposed Q4_K
// down: one workgroup of 8 wavefronts per unit, a (token, pair) of the
// request (units b, b+G, ...), so that no h crosses workgroups.
//
// Gate and up run on the matrix cores, exactly in integers. Each value of x
// is written as four signed 8-bit digits over a power of two per 32-value
// sub-block, x = 2^e (2^24 d0 + 2^16 d1 + 2^8 d2 + d3) with |x| 2^-e < 2^30
// (31 bits relative to the sub-block's largest value, below fp32 rounding:
// a staging error is the same for every row, so it adds up coherently in y).
// One 16x16x64 int8 product takes 16 rows (gate and up of 8 neurons), 16
// values of each of 4 sub-blocks as k, and 16 columns (sub-block, digit); columns whose
// sub-block is not that of the k range are zero, so that after the two
// products of a group C[row][(s, d)] is the exact integer dot of row and
// digit d over sub-block s. Each lane then scales its 4 values by
// d*sc (fp32, as the reference forms it, src/native.c:14-19) times 2^e
// times the digit's weight and adds them to its row sums; the min term is
// dmin*m times the fp32 sum of the sub-block's x. Wavefront w owns
// super-blocks 2w and 2w+1 of every row.
//
// A unit is processed in 4 rounds, one row-block (8 neurons) each: the
// round's row sums meet in LDS behind a barrier, and every wavefront forms
// the round's 8 h = SiLU(a)*u in fp32 (backends/ref.c:82-83) itself. The
// down projection is the fp32 one, one round late: each wavefront builds
// d*sc*gate*h and dmin*m*gate*h of the round's neurons for its two
// super-blocks of outputs (512w..512w+511) and accumulates 8 outputs per
// lane. A second small kernel on the same stream, decode_reduce, sums the
// unit partials in unit order: the kernel boundary is the global barrier and
// makes the partials visible across XCDs.
//
// Every lane loads the bytes it uses into registers with the default cache
// policy (measured faster here than the non-temporal one, and it lets the
// units of one pair that follow each other in a workgroup's chunk find its
// bytes cached), one round ahead: round r+1's gate/up and down bytes during round r
// (the next unit's headers and first round during round 3). One round in
// flight (about 55 KB per workgroup) streams at the measured ceiling; two
// rounds in flight stream more slowly.

// The weight loads are raw buffer loads: the pair's slice is a buffer
// resource in scalar registers (bounded by the slice's bytes, so that an
// offset past it reads zeros), the per-lane part of each offset is computed
// once, the per-load part is a scalar offset. No 64-bit address arithmetic
// per load, and the loads count in vmcnt only.
struct PairBuf {
  __amdgpu_buffer_rsrc_t rsrc;         // the pair's slice
  uint32_t proj;                       // bytes of the 32 gate rows (= up offset)
  float gate;                          // the token's expert weight
  uint32_t token;                      // the unit's token
};
// The fields pass through readfirstlane: they are uniform (one pair per
// workgroup at a time), and the compiler must know it, or it would wrap every
// buffer load in a loop over distinct resource values.
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
// Plan reads through the constant address space: the plan is read-only
// while the kernel runs, so they become scalar loads, which count in the
// scalar counter. A vector load of a descriptor would make its wait also
// wait for every weight load issued before it.
__device__ __forceinline__ uint32_t plan_read(const uint32_t* p) {
  return *(const __attribute__((address_space(4))) uint32_t*)p;
}
template <class T>
__device__ __forceinline__ uint32_t plan_field(const T* base, size_t offset) {
  return plan_read(reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(base) + offset));
}
// The descriptor's words are read whole (the token is the top byte of the
// word of its four byte fields): scalar loads have no byte form.
// With `live` false the resource has no records: its loads return zeros
// without a memory access (the requests past a workgroup's last unit).
__device__ __forceinline__ PairBuf pair_buf(const PairDesc* P, bool live = true) {
  static_assert(offsetof(PairDesc, gu) == 12 && offsetof(PairDesc, pad) == 15, "descriptor word 3");
  PairBuf B;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(P);
  const uint64_t base = ((uint64_t)uniform(plan_read(w + 1)) << 32) | uniform(plan_read(w));
  B.token = uniform(plan_read(w + 3)) >> 24;
  B.proj = uniform(plan_read(w + 2));
  B.gate = __uint_as_float(uniform(plan_read(reinterpret_cast<const uint32_t*>(P->gate))));
  B.rsrc = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), (short)0, live ? (int)(3 * B.proj) : 0,
                                              0x00020000);
  return B;
}
__device__ __forceinline__ uint4 bld(const PairBuf& B, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(B.rsrc, (int)voff, (int)soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

constexpr int kSubBlocks = kMaxHidden / 32;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct DecodeDnBytes {                 // one lane's down bytes of one round
  uint4 dq[2];                         // nibbles: super-block 2w + l/32, neurons 8r..8r+7,
                                       // outputs 8j..8j+3 and 8j+4..8j+7 (j = l%32)
  uint4 dh;                            // header: super-block 2w + (l%16)/8, neuron 8r + l%8
};
struct DecodeTable {                   // one wavefront's down coefficients of one round
  float D[2][8][8];                    // [super-block][group][neuron] d*sc*gate*h
  float M[2][8][8];                    // dmin*mi*gate*h
};
struct DecodeLds {
  int8_t xd[2][4][kSubBlocks][32];           // [unit parity][digit][sub-block][value]: x of the unit's token
  float xf[2][kSubBlocks];                   // 2^e of each sub-block
  float xs[2][kSubBlocks];                   // fp32 sum of each sub-block's values
  float dsc[kDecodeWaves][16][64];           // [wave][sub-block of its super-blocks][row] d*sc
  float rowp[2][kDecodeWaves][64];           // [unit parity][wave][row] scaled integer dots
  float minp[2][kDecodeWaves][64];           // [unit parity][wave][row] min terms
  float h[kDecodeWaves][8];                  // gate*h of the round (each wavefront's own copy)
  uint4 dh[kDecodeWaves][16];                // [wave][super-block 2w + i/8, neuron 8r + i%8]
  DecodeTable table[kDecodeWaves];
};
static_assert(sizeof(DecodeLds) <= 160 * 1024, "decode LDS");

// Round (row-block) rb of the unit's gate/up nibbles for this wavefront's
// super-blocks 2w, 2w+1: [super-block][part], lane l's 16 bytes.
struct DecodeNib {
  uint4 q[2][2];
};
// sb0, sb1 are clamped to the matrix by the caller; every load is issued,
// so that the compiler's waits count all of them.
__device__ __forceinline__ void load_nib(const PairBuf& B, unsigned rb, unsigned sb0, unsigned sb1, int lane,
                                         DecodeNib& N) {
  const uint32_t v = 16 * (uint32_t)lane;
#pragma unroll
  for (int sbl = 0; sbl < 2; ++sbl)
#pragma unroll
    for (int p = 0; p < 2; ++p) N.q[sbl][p] = bld(B, v, 9216 * (sbl ? sb1 : sb0) + 1024 + 2048 * rb + 1024 * p);
}
// Headers of super-block sb: lane l holds row l (row-block l/16, row l%16).
__device__ __forceinline__ uint4 load_hdr(const PairBuf& B, unsigned sb, int lane) {
  return bld(B, 16 * (uint32_t)lane, 9216 * sb);
}
// Round r of the down matrix: the lane's nibbles of neurons 8r..8r+7 and one
// header (dq: 4608 * super-block + 32 * (l%32); dh: + 4096 + 16 * (l%8)).
__device__ __forceinline__ void load_dn(const PairBuf& B, unsigned r, uint32_t dq, uint32_t dh, DecodeDnBytes& R) {
  const uint32_t base = 2 * B.proj;
  R.dq[0] = bld(B, dq, base + 1024 * r);
  R.dq[1] = bld(B, dq + 16, base + 1024 * r);
  R.dh = bld(B, dh, base + 128 * r);
}

// x of a token into digits in slot `slot` (thread: sub-block tid/4, values
// 8*(tid%4)..+7, from v). The four threads of a sub-block agree on its
// largest magnitude and sum through butterflies within their quad. With
// kLanes the digits go to the lane-major layout of the row-format kernel,
// xl[digit][j][k][c]: values 16k..16k+15 of sub-block 2c + j, so that lane c
// reads its two sub-blocks' 16-byte pieces next to lanes c-1 and c+1.
template <class Lds, bool kLanes = false>
__device__ __forceinline__ void stage_x(const float4 (&v4)[2], unsigned slot, unsigned nsub, bool routed, Lds& L,
                                        uint32_t& bad) {
  const unsigned tid = threadIdx.x, s = tid >> 2, q = tid & 3;
  const float v[8] = {v4[0].x, v4[0].y, v4[0].z, v4[0].w, v4[1].x, v4[1].y, v4[1].z, v4[1].w};
  float m = 0.f;
  uint32_t fin = 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m = fmaxf(m, fabsf(v[i]));
    fin &= isfinite(v[i]) ? 1u : 0u;
  }
  float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  fin &= (uint32_t)__shfl_xor((int)fin, 1);
  fin &= (uint32_t)__shfl_xor((int)fin, 2);
  if (!fin && routed && s < nsub) bad |= kErrRange;   // a non-finite x makes every a of the token non-finite
  int E = 0;
  if (m > 0.f) (void)frexpf(m, &E);                  // m < 2^E
  const int e = max(E - 30, -149);
  uint32_t w[4][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int X = fin ? (int)rintf(ldexpf(v[i], -e)) : 0;   // |X| <= 2^30
    const int d3 = ((X + 128) & 255) - 128, X1 = (X - d3) >> 8;
    const int d2 = ((X1 + 128) & 255) - 128, X2 = (X1 - d2) >> 8;
    const int d1 = ((X2 + 128) & 255) - 128, d0 = (X2 - d1) >> 8;   // |d0| <= 65
    w[0][i >> 2] |= (uint32_t)(d0 & 255) << (8 * (i & 3));
    w[1][i >> 2] |= (uint32_t)(d1 & 255) << (8 * (i & 3));
    w[2][i >> 2] |= (uint32_t)(d2 & 255) << (8 * (i & 3));
    w[3][i >> 2] |= (uint32_t)(d3 & 255) << (8 * (i & 3));
  }
  if (s < nsub) {
    if constexpr (kLanes) {
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<uint2*>(&L.xl[d][s & 1][q >> 1][s >> 1][2 * (q & 1)]) = make_uint2(w[d][0], w[d][1]);
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) *reinterpret_cast<uint2*>(&L.xd[slot][d][s][8 * q]) = make_uint2(w[d][0], w[d][1]);
    }
    if (q == 0) {
      L.xf[slot][s] = ldexpf(1.f, e);
      L.xs[slot][s] = sum;
    }
  }
}

// Headers of super-block sb (sbl = sb - 2w) into this wavefront's d*sc
// table; returns the row's min term over the super-block.
__device__ __forceinline__ float header_pass(const uint4& h, unsigned sb, unsigned sbl, unsigned t, int wave, int lane,
                                             DecodeLds& L, uint32_t& bad) {
  if (half_bad(h.x) || half_bad(h.x >> 16)) bad |= kErrScale;
  const float d = half_to_float(h.x & 0xffff), dm = half_to_float(h.x >> 16);
  // q4k_scale_min for all eight sub-blocks at once, one value per byte:
  // sub-blocks 0..3 are the low six bits of bytes 0..3 (scales) and 4..7
  // (mins); sub-blocks 4..7 take the low (scales) or high (mins) nibble of
  // bytes 8..11 with the top two bits of bytes 0..3 or 4..7 above it.
  const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, mi_lo = h.z & 0x3F3F3F3Fu;
  const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
  const uint32_t mi_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  float mins = 0.f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const float sc = ub(g < 4 ? sc_lo : sc_hi, g & 3), mi = ub(g < 4 ? mi_lo : mi_hi, g & 3);
    L.dsc[wave][8 * sbl + g][lane] = d * sc;
    mins += (dm * mi) * L.xs[t][8 * sb + g];   // t: the x slot
  }
  return mins;
}

// The x operands of super-block sb (x slot t): lane (kg = l/16, column
// j = l%16 = 4 * sub-block + digit) holds digit j%4 of values 16hh..16hh+15
// of sub-block 4G + kg for product m = 2G + hh when its column's sub-block
// is kg, zero otherwise; fx[G] = 2^e * digit weight of its column's sub-block.
template <class Lds>
__device__ __forceinline__ void x_operands(unsigned t, unsigned sb, int lane, const Lds& L, i32x4 (&b)[4],
                                           float (&fx)[2]) {
  const unsigned kg = (unsigned)lane >> 4, j = (unsigned)lane & 15, js = j >> 2, jd = j & 3;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned G = (unsigned)m >> 1, hh = (unsigned)m & 1;
    const i32x4 z = {0, 0, 0, 0};
    b[m] = js == kg ? *reinterpret_cast<const i32x4*>(&L.xd[t][jd][8 * sb + 4 * G + kg][16 * hh]) : z;
  }
  const float wd = jd == 0 ? 16777216.f : jd == 1 ? 65536.f : jd == 2 ? 256.f : 1.f;
#pragma unroll
  for (int G = 0; G < 2; ++G) fx[G] = L.xf[t][8 * sb + 4 * G + js] * wd;
}

// Row-block rb of super-block 2w + sbl: two products per group of four
// sub-blocks, then each lane's four values scaled into acc (rows 4kg..4kg+3).
__device__ __forceinline__ void rb_products(const uint4 (&q)[2], const i32x4 (&b)[4], const float (&fx)[2],
                                            unsigned sbl, unsigned rb, int wave, int lane, const DecodeLds& L,
                                            float (&acc)[4]) {
  const unsigned kg = (unsigned)lane >> 4, js = ((unsigned)lane & 15) >> 2;
#pragma unroll
  for (int G = 0; G < 2; ++G) {
    const uint4 w = q[G];
    i32x4 c = {0, 0, 0, 0};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint32_t w0 = hh ? w.z : w.x, w1 = hh ? w.w : w.y;
      const i32x4 a = {(int)nib_lo(w0), (int)nib_hi(w0), (int)nib_lo(w1), (int)nib_hi(w1)};
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[2 * G + hh], c, 0, 0, 0);
    }
    const float4 ds = *reinterpret_cast<const float4*>(&L.dsc[wave][8 * sbl + 4 * G + js][16 * rb + 4 * kg]);
    acc[0] = fmaf((float)c[0], ds.x * fx[G], acc[0]);
    acc[1] = fmaf((float)c[1], ds.y * fx[G], acc[1]);
    acc[2] = fmaf((float)c[2], ds.z * fx[G], acc[2]);
    acc[3] = fmaf((float)c[3], ds.w * fx[G], acc[3]);
  }
}

// SiLU(a)*u in fp32 with the stable sigmoid form; a, u or h outside fp32
// is the reference's FR_NUMERIC (backends/ref.c:37-40).
__device__ __forceinline__ float silu_mul_f32(float a, float u, uint32_t& bad) {
  const float e = __expf(-fabsf(a));
  const float inv = __builtin_amdgcn_rcpf(1.f + e);
  const float sig = a >= 0.f ? inv : e * inv;
  const float h = a * sig * u;
  if (!isfinite(a) || !isfinite(u) || !isfinite(h)) {
    bad |= kErrRange;
    return 0.f;
  }
  return h;
}

// Down projection of round r (neurons 8r..8r+7, gate*h in hs[0..7]) from the
// round's down bytes: coefficients, then 8 outputs per lane.
__device__ __forceinline__ void down_round(const DecodeDnBytes& R, const float* hs, int wave, int lane, unsigned nsb,
                                           DecodeLds& L, float (&y)[8], uint32_t& bad) {
  if (lane < 16) L.dh[wave][lane] = R.dh;
  DecodeTable& T = L.table[wave];
  {
    // Lane (s, group, neurons 2q, 2q+1) of this wavefront's two super-blocks.
    const unsigned ts = (unsigned)lane >> 5, tg = ((unsigned)lane >> 2) & 7, n0 = 2 * ((unsigned)lane & 3);
    const bool tvalid = 2 * (unsigned)wave + ts < nsb;
    float Dv[2], Mv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4 hdr = L.dh[wave][8 * ts + n0 + q];
      bool ok;
      hdr_dm(hdr, tg, Dv[q], Mv[q], ok);
      if (tvalid && !ok) bad |= kErrScale;
      const float gh = hs[n0 + q];
      Dv[q] *= gh * kFp8Nibble;   // the nibbles below are q * 2^-9
      Mv[q] *= gh;
    }
    *reinterpret_cast<float2*>(&T.D[ts][tg][n0]) = make_float2(Dv[0], Dv[1]);
    *reinterpret_cast<float2*>(&T.M[ts][tg][n0]) = make_float2(Mv[0], Mv[1]);
  }
  __builtin_amdgcn_wave_barrier();
  const unsigned sbl = (unsigned)lane >> 5, j = (unsigned)lane & 31, g = j >> 2;   // 8 outputs
  if (2 * (unsigned)wave + sbl < nsb) {
    const float4* cd = reinterpret_cast<const float4*>(&T.D[sbl][g][0]);
    const float4* cm = reinterpret_cast<const float4*>(&T.M[sbl][g][0]);
    const float4 d0 = cd[0], d1 = cd[1], m0 = cm[0], m1 = cm[1];
    const float coef[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
    const float msum = ((m0.x + m0.y) + (m0.z + m0.w)) + ((m1.x + m1.y) + (m1.z + m1.w));
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint4 dq = R.dq[half];
      float s4[4] = {-msum, -msum, -msum, -msum};
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        // Dword wd: neurons 2wd (bytes 0,1) and 2wd+1 (bytes 2,3); low
        // nibbles columns 0 and 2, high nibbles columns 1 and 3.
        const uint32_t v = word(dq, wd);
        const uint32_t lo = nib_lo(v), hi = nib_hi(v);
        const float2 la = nib_pair<false>(lo), lb = nib_pair<true>(lo), ha = nib_pair<false>(hi), hb = nib_pair<true>(hi);
        const float ca = coef[2 * wd], cb = coef[2 * wd + 1];
        s4[0] = fmaf(la.x, ca, s4[0]);
        s4[1] = fmaf(ha.x, ca, s4[1]);
        s4[2] = fmaf(la.y, ca, s4[2]);
        s4[3] = fmaf(ha.y, ca, s4[3]);
        s4[0] = fmaf(lb.x, cb, s4[0]);
        s4[1] = fmaf(hb.x, cb, s4[1]);
        s4[2] = fmaf(lb.y, cb, s4[2]);
        s4[3] = fmaf(hb.y, cb, s4[3]);
      }
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) y[4 * half + cc] += s4[cc];
    }
  }
  __builtin_amdgcn_wave_barrier();   // the table and headers are read before the next round writes them
}

// Unit partials, [position block][unit][16 positions]: position p of unit u
// at float (p/16 * stride + u) * 16 + p%16 (stride: units per block), so
// that decode_reduce's workgroup for one block of 16 positions reads its
// units' values as one contiguous run.
__device__ __forceinline__ size_t partial_index(unsigned unit, unsigned p, unsigned stride) {
  return ((size_t)(p >> 4) * stride + unit) * 16 + (p & 15);
}

// The unit's fp32 partial: wavefront w, half h, lane l -> positions
// 4*(128w + 64h + l)..+3, columns 256*sb + 8j + 4h..+3 (sb = 2w + l/32,
// j = l%32), four lanes to a 64-byte piece; y restarts at 0. The kernel
// boundary makes the partials visible to decode_reduce.
__device__ __forceinline__ void store_partial(float* wgpart, unsigned stride, unsigned unit, int wave, int lane,
                                              float (&y)[8]) {
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
    *reinterpret_cast<float4*>(wgpart + partial_index(unit, 4 * (128 * wave + 64 * hh + lane), stride)) =
        make_float4(y[4 * hh], y[4 * hh + 1], y[4 * hh + 2], y[4 * hh + 3]);
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = 0.f;
}

// The status word the decode kernels flag errors into, and block 0's
// set-up: the engine's launches clear the next launch's parity; a static
// launch zeroes the caller's status word (which only decode_reduce, a later
// kernel, writes) and flags into the static error word, which decode_reduce
// folds into it and zeroes again.
__device__ __forceinline__ uint32_t* decode_status(const Scratch& S) {
  if (blockIdx.x == 0) {
    if (S.ystat) {
      if (threadIdx.x == 0) *S.ystat = 0;
    } else if (!S.hstat) {
      clear_other_parity(S);
    }
  }
  return S.ystat || S.hstat ? S.dstat : S.out + (size_t)S.parity * S.out_words;
}

__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + S.A.pairs_off);
  const unsigned hidden = S.A.hidden, nsb = hidden / 256, nsub = hidden / 32;
  const unsigned np = S.A.npairs, tpw = S.A.tpw;
  const unsigned burst = S.A.burst;
  // Token-major partial index of each unit of the work list (after the token table).
  const uint32_t* upart = reinterpret_cast<const uint32_t*>(plan + S.A.groups_off + burst * sizeof(DecodeToken));
  // The wavefront index through readfirstlane: the compiler then knows it is
  // uniform, so offsets built from it stay in scalar registers.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) DecodeLds L;
  const float* xg = reinterpret_cast<const float*>(plan + S.A.x_off);
  const unsigned xs0 = 32 * ((unsigned)tid >> 2) + 8 * ((unsigned)tid & 3);   // this thread's 8 values of a token
  const bool xin = ((unsigned)tid >> 2) < nsub;
  const unsigned sb0 = 2 * (unsigned)wave, sb1 = sb0 + 1;
  const bool has0 = sb0 < nsb, has1 = sb1 < nsb;
  const unsigned lb0 = min(sb0, nsb - 1), lb1 = min(sb1, nsb - 1);   // super-blocks loaded (clamped)
  // Down-matrix offsets of this lane (super-blocks clamped to the matrix).
  const uint32_t dq_off = 4608 * min(2 * (unsigned)wave + ((unsigned)lane >> 5), nsb - 1) + 32 * ((unsigned)lane & 31);
  const uint32_t dh_off =
      4608 * min(2 * (unsigned)wave + (((unsigned)lane & 15) >> 3), nsb - 1) + 4096 + 16 * ((unsigned)lane & 7);
  uint32_t bad = 0;

  // The first unit's x is requested first, then its round 0, so that waiting
  // for x does not wait for the weights. x is staged per unit (the units of
  // a burst are token-major): the next unit's x is requested with its first
  // bytes and staged into the other slot after this unit.
  unsigned p = blockIdx.x * tpw;   // this workgroup's chunk: units [p, min(p + tpw, np))
  const unsigned pend = min(p + tpw, np);
  // A single-token plan's x is token 0's: requested before the descriptor.
  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  if (burst == 1 && xin) {
    xv[0] = *reinterpret_cast<const float4*>(xg + xs0);
    xv[1] = *reinterpret_cast<const float4*>(xg + xs0 + 4);
  }
  PairBuf B = pair_buf(pairs + p);
  if (burst != 1 && xin) {
    const float* xt = xg + (size_t)B.token * hidden + xs0;
    xv[0] = *reinterpret_cast<const float4*>(xt);
    xv[1] = *reinterpret_cast<const float4*>(xt + 4);
  }
  uint4 h0 = make_uint4(0u, 0u, 0u, 0u), h1 = h0;
  DecodeNib N[4];                      // [round]: round r+1's bytes are in flight during round r
  DecodeDnBytes D[4];                  // a round's down bytes are used one round later (lagged down)
  h0 = load_hdr(B, lb0, lane);
  h1 = load_hdr(B, lb1, lane);
  load_nib(B, 0, lb0, lb1, lane, N[0]);
  load_dn(B, 0, dq_off, dh_off, D[0]);
  __builtin_amdgcn_sched_barrier(0);
  stage_x(xv, 0, nsub, true, L, bad);
  __syncthreads();   // x is in LDS

  float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const unsigned kg = (unsigned)lane >> 4, jcol = (unsigned)lane & 15;
  // Unit k: round rb = 0..3 requests round rb+1's bytes (the next unit's
  // headers and round 0 after round 3), applies the down projection of round
  // rb-1 (its bytes and h are at hand), forms row-block rb's gate/up sums,
  // meets the other wavefronts at the barrier and forms the round's 8 h;
  // round 3's down follows the loop. Doing the lagged down first gives the
  // round's gate/up bytes that much longer to arrive. The scheduling
  // barriers keep the loads where they are written. Round 1's bytes are
  // requested before the header pass, whose wait on the headers would
  // otherwise delay them.
  for (unsigned k = 0;; ++k) {
    const unsigned q = p + 1, par = k & 1, t = par;   // t: this unit's x slot
    const bool more = q < pend;
    const PairBuf Bn = pair_buf(pairs + (more ? q : p), more);
    load_nib(B, 1, lb0, lb1, lane, N[1]);
    load_dn(B, 1, dq_off, dh_off, D[1]);
    __builtin_amdgcn_sched_barrier(0);
    i32x4 b0[4], b1[4];
    float fx0[2], fx1[2];
    x_operands(t, sb0, lane, L, b0, fx0);
    x_operands(t, sb1, lane, L, b1, fx1);
    {
      float mp = 0.f;
      if (has0) mp += header_pass(h0, sb0, 0, t, wave, lane, L, bad);
      if (has1) mp += header_pass(h1, sb1, 1, t, wave, lane, L, bad);
      L.minp[par][wave][lane] = mp;
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const DecodeNib& Nc = N[rb];
      __builtin_amdgcn_sched_barrier(0);
      if (rb == 1 || rb == 2) {
        load_nib(B, rb + 1, lb0, lb1, lane, N[rb + 1]);
        load_dn(B, rb + 1, dq_off, dh_off, D[rb + 1]);
      } else if (rb == 3) {   // the next unit (zeros without a memory access after the last)
        if (xin) {
          const float* xt = xg + (size_t)Bn.token * hidden + xs0;
          xv[0] = *reinterpret_cast<const float4*>(xt);
          xv[1] = *reinterpret_cast<const float4*>(xt + 4);
        }
        h0 = load_hdr(Bn, lb0, lane);
        h1 = load_hdr(Bn, lb1, lane);
        load_nib(Bn, 0, lb0, lb1, lane, N[0]);
        load_dn(Bn, 0, dq_off, dh_off, D[0]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (rb) down_round(D[rb - 1], L.h[wave], wave, lane, nsb, L, y, bad);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      if (has0) rb_products(Nc.q[0], b0, fx0, 0, rb, wave, lane, L, acc);
      if (has1) rb_products(Nc.q[1], b1, fx1, 1, rb, wave, lane, L, acc);
      {
        float4 v4;
        v4.x = row_sum(acc[0]);
        v4.y = row_sum(acc[1]);
        v4.z = row_sum(acc[2]);
        v4.w = row_sum(acc[3]);
        if (jcol == 0) *reinterpret_cast<float4*>(&L.rowp[par][wave][16 * rb + 4 * kg]) = v4;
      }
      __syncthreads();   // every wavefront's sums of row-block rb are in LDS
      // h of neurons 8rb..8rb+7 (gate row 16rb + i, up row 16rb + 8 + i);
      // every wavefront forms its own copy.
      if (lane < 8) {
        const unsigned rg = 16 * rb + (unsigned)lane, ru = rg + 8;
        float a = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
          a += L.rowp[par][w][rg] - L.minp[par][w][rg];
          u += L.rowp[par][w][ru] - L.minp[par][w][ru];
        }
        uint32_t hb = 0;
        const float gh = B.gate * silu_mul_f32(a, u, hb);
        if (wave == 0) bad |= hb;
        L.h[wave][lane] = gh;
      }
      __builtin_amdgcn_wave_barrier();
    }
    down_round(D[3], L.h[wave], wave, lane, nsb, L, y, bad);
    store_partial(S.wgpart, S.ustride, plan_read(upart + p), wave, lane, y);
    if (!more) break;
    stage_x(xv, par ^ 1, nsub, true, L, bad);
    __syncthreads();   // the next unit's x is in LDS
    p = q;
    B = Bn;
  }
  if (bad) flag(status, bad);
}

// ------------------------------------------------- decode kernel, split units
//
// decode_kernel gives each unit to one workgroup, whose CU streams the
// unit's 221 KB: when a node owns few blocks a request has few units, most
// CUs idle, and a call takes as long as a full layer share. Here each unit
// is split into `split` items of 4/split row-blocks (split 4 for at most 5
// owned blocks, 2 for at most 11): an item computes its row-blocks' gate/up
// and h as decode_kernel's rounds do, then the down of those neurons over
// every output into a partial of its own, and decode_reduce sums a token's
// items in (unit, item) order. The split depends on the owned blocks only,
// so a burst row and the same token run alone split the same way and stay
// bit-identical. All of an item's bytes are requested at once (x, headers,
// one or two rounds). kRounds: row-blocks per item (1 for split 4, 2 for
// split 2).
template <unsigned kRounds>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  const PlanHeader* PH = reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + plan_field(PH, offsetof(PlanHeader, pairs_off)));
  const unsigned hidden = plan_field(PH, offsetof(PlanHeader, hidden)), nsb = hidden / 256, nsub = hidden / 32;
  const unsigned np = plan_field(PH, offsetof(PlanHeader, npairs)), tpw = plan_field(PH, offsetof(PlanHeader, tpw));
  const unsigned burst = plan_field(PH, offsetof(PlanHeader, burst));
  constexpr unsigned split = 4 / kRounds;
  const uint32_t* upart = reinterpret_cast<const uint32_t*>(plan + plan_field(PH, offsetof(PlanHeader, groups_off)) +
                                                          burst * sizeof(DecodeToken));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) DecodeLds L;
  const float* xg = reinterpret_cast<const float*>(plan + plan_field(PH, offsetof(PlanHeader, x_off)));
  const unsigned xs0 = 32 * ((unsigned)tid >> 2) + 8 * ((unsigned)tid & 3);
  const bool xin = ((unsigned)tid >> 2) < nsub;
  const unsigned sb0 = 2 * (unsigned)wave, sb1 = sb0 + 1;
  const bool has0 = sb0 < nsb, has1 = sb1 < nsb;
  const unsigned lb0 = min(sb0, nsb - 1), lb1 = min(sb1, nsb - 1);
  const uint32_t dq_off = 4608 * min(2 * (unsigned)wave + ((unsigned)lane >> 5), nsb - 1) + 32 * ((unsigned)lane & 31);
  const uint32_t dh_off =
      4608 * min(2 * (unsigned)wave + (((unsigned)lane & 15) >> 3), nsb - 1) + 4096 + 16 * ((unsigned)lane & 7);
  const unsigned kg = (unsigned)lane >> 4, jcol = (unsigned)lane & 15;
  uint32_t bad = 0;
  const unsigned items = np * split, iend = min((blockIdx.x + 1) * tpw, items);
  for (unsigned it = blockIdx.x * tpw; it < iend; ++it) {
    const unsigned p = it / split, part = it % split, rb0 = kRounds * part;
    const PairBuf B = pair_buf(pairs + p);
    float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
    if (xin) {
      const float* xt = xg + (size_t)B.token * hidden + xs0;
      xv[0] = *reinterpret_cast<const float4*>(xt);
      xv[1] = *reinterpret_cast<const float4*>(xt + 4);
    }
    const uint4 h0 = load_hdr(B, lb0, lane), h1 = load_hdr(B, lb1, lane);
    DecodeNib N[kRounds];
    DecodeDnBytes D[kRounds];
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
      load_nib(B, rb0 + r, lb0, lb1, lane, N[r]);
      load_dn(B, rb0 + r, dq_off, dh_off, D[r]);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();   // every wavefront is past the previous item's reads of x, the tables and h
    stage_x(xv, 0, nsub, true, L, bad);
    __syncthreads();   // x is in LDS
    i32x4 b0[4], b1[4];
    float fx0[2], fx1[2];
    x_operands(0, sb0, lane, L, b0, fx0);
    x_operands(0, sb1, lane, L, b1, fx1);
    {
      float mp = 0.f;
      if (has0) mp += header_pass(h0, sb0, 0, 0, wave, lane, L, bad);
      if (has1) mp += header_pass(h1, sb1, 1, 0, wave, lane, L, bad);
      L.minp[0][wave][lane] = mp;
    }
    float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
      const unsigned rb = rb0 + r;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      if (has0) rb_products(N[r].q[0], b0, fx0, 0, rb, wave, lane, L, acc);
      if (has1) rb_products(N[r].q[1], b1, fx1, 1, rb, wave, lane, L, acc);
      {
        float4 v4;
        v4.x = row_sum(acc[0]);
        v4.y = row_sum(acc[1]);
        v4.z = row_sum(acc[2]);
        v4.w = row_sum(acc[3]);
        if (jcol == 0) *reinterpret_cast<float4*>(&L.rowp[0][wave][16 * rb + 4 * kg]) = v4;
      }
      __syncthreads();   // every wavefront's sums of row-block rb are in LDS
      if (lane < 8) {
        const unsigned rg = 16 * rb + (unsigned)lane, ru = rg + 8;
        float a = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
          a += L.rowp[0][w][rg] - L.minp[0][w][rg];
          u += L.rowp[0][w][ru] - L.minp[0][w][ru];
        }
        uint32_t hb = 0;
        const float gh = B.gate * silu_mul_f32(a, u, hb);
        if (wave == 0) bad |= hb;
        L.h[wave][lane] = gh;
      }
      __builtin_amdgcn_wave_barrier();
      down_round(D[r], L.h[wave], wave, lane, nsb, L, y, bad);
    }
    store_partial(S.wgpart, S.ustride, plan_read(upart + p) * split + part, wave, lane, y);
  }
  if (bad) flag(status, bad);
}

// ------------------------------------------------- decode kernel, bursts
//
// F32, a burst of two or more tokens, every pair Q4_K gate/up (TQ4_KM tiles)
// with the transposed Q4_K down, routed experts only, on a node that owns 12
// or more blocks: one workgroup turn per unique (expert, block) pair, which
// computes every token that routes to it at once. The pair's bytes are read
// once, and the tokens sit in the columns of f16 matrix-core products, so a
// token costs a column of each product instead of a pass of its own.
//
// Columns: token t in column 2t (hi part of its operand) and 2t+1 (lo part).
// Gate/up, per super-block and row-block: A = sc*q, the 6-bit sub-block scale
// times the nibble (< 1024), exactly in f16 (nib_pair_sc: the nibble bytes
// as FP8 E4M3 scaled by 2^9, then a packed f16 multiply by sc);
// lane 16kg + i holds row i, sub-block 4p + kg, as the TQ4_KM tiles lie, so
// one v_mfma_f32_16x16x32_f16 spans 8 positions of 4 sub-blocks and 8 of them
// the super-block. B = x' of the column's token, x' = x*2^-e with |x'| < 2^15
// over the token's values in the super-block, as hi = f16(x'), lo = f16(x' -
// hi) (22 significant bits). The super-block's sums are scaled once by
// d*2^e; the min terms -dmin*m*sum(x) take v_mfma_f32_16x16x4f32 per
// four sub-blocks on the fp32 sub-block sums of x. x is staged once per
// workgroup: each wavefront turns its own two super-blocks of every token
// into B operands that stay in registers for all of its pairs.
//
// Down, after the fourth round, per tile of 16 outputs (inside one 32-output
// sub-block): A = sc*q of the 16 outputs x 32 neurons (each neuron's scale of
// that sub-block), B = d*gate*h of each neuron and column in two f16 parts
// over a power of two per (super-block, token). The min terms
// -dmin*m*gate*h are one more product per sub-block (A = m, the same for
// every output of the sub-block) that starts its two tiles' accumulators.
// The 16-byte down units hold 4 outputs x 8 neurons; lane 16kg + 4a + q loads
// the unit its quad needs for tile 4G + q, the quad shares it by DPP
// broadcast, and each lane takes its own output q.
//
// Partials: one per (token, pair), in decode_kernel's position layout and
// token-major numbering, which decode_reduce sums in the reference's order.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
struct BurstLds {
  // Rows are padded so that the 8 tokens' 16-byte pieces fall on distinct banks.
  float rowp[4][kDecodeWaves][kMaxBurst][20];   // [round][wave][token][row]: each wavefront's row sums
  float h[kMaxBurst][kNeurons + 4];             // [token][neuron] gate*h of the pair
  uint4 hdr[kDecodeWaves][2][64];               // [wave][super-block][row-block*16 + row]: gate/up headers
  float dg[kDecodeWaves][2][64];                // d of each gate/up header
  uint4 dsc[kDecodeWaves][2][8][4];             // [wave][super-block][sub-block][kg]: down sc of neurons 8kg.. as u16
  uint4 dmn[kDecodeWaves][2][8][4];             // the down mins, same layout, as f16
  float dd[kDecodeWaves][2][kNeurons];          // [wave][super-block][neuron] down d
  float dm[kDecodeWaves][2][kNeurons];          // down dmin
  float out[kDecodeWaves][kMaxBurst][260];      // [wave][token][output]: one super-block's down outputs (unscaled)
};
// x of up to 4 tokens at a time, staged by the whole workgroup: per token
// and part a row of 4096 f16 values (16 bytes of padding between rows, so
// that the 16 lanes of a 16-byte read hit distinct banks), 2^e per
// (token, super-block) and the fp32 sum of each 32-value sub-block.
constexpr int kStageTokens = 4;
constexpr int kStageRow = kMaxHidden + 8;   // f16 values per (token, part) row
struct BurstStage {
  _Float16 x[kStageTokens * 2][kStageRow];
  int e[kStageTokens][kMaxHidden / 256];
  float sum[kStageTokens][kSubBlocks];
};
union BurstShared {
  BurstStage stage;   // before the first pair
  BurstLds pair;      // from the first pair on
};
static_assert(sizeof(BurstShared) <= 160 * 1024, "burst LDS");

// A round's gate/up nibbles of the wavefront's two super-blocks,
// [super-block][part] (lane 16kg + i: row i, sub-block 4 part + kg).
struct BurstRound {
  uint4 q[2][2];
};
__device__ __forceinline__ void load_burst_round(const PairBuf& B, unsigned rb, unsigned lb0, unsigned lb1, int lane,
                                                 BurstRound& R) {
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int p = 0; p < 2; ++p)
      R.q[s][p] = bld(B, 16 * (uint32_t)lane, 9216 * (s ? lb1 : lb0) + 1024 + 2048 * rb + 1024 * p);
}
// The pair's gate/up headers of the two super-blocks: lane l holds the
// 16-byte header of row l%16 of row-block l/16.
struct BurstHdr {
  uint4 h[2];
};
__device__ __forceinline__ void load_burst_hdr(const PairBuf& B, unsigned lb0, unsigned lb1, int lane, BurstHdr& H) {
  H.h[0] = bld(B, 16 * (uint32_t)lane, 9216 * lb0);
  H.h[1] = bld(B, 16 * (uint32_t)lane, 9216 * lb1);
}
// The down bytes: unit (kg, 4(4G + q) + a) of each super-block for lane
// 16kg + 4a + q (the unit its quad needs for tile 4G + q), and the header of
// neuron l%32 of super-block 2w + l/32 (voff_h carries the super-block).
struct BurstDown {
  uint4 u[2][4];
  uint4 h;
};
__device__ __forceinline__ void load_burst_down(const PairBuf& B, unsigned lb0, unsigned lb1, uint32_t voff_u,
                                                uint32_t voff_h, BurstDown& D) {
  const uint32_t base = 2 * B.proj;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int G = 0; G < 4; ++G) D.u[s][G] = bld(B, voff_u, base + 4608 * (s ? lb1 : lb0) + 256 * G);
  D.h = bld(B, voff_h, base + 4096);
}

// Two nibble values (u16 halves of p, each below 16) times the 6-bit scale
// (sc2 = sc | sc << 16) as two f16 in one dword: the packed 16-bit
// multiply-add forms the f16 bits of 1024 + sc*q (exact: sc*q < 1024), and
// subtracting 1024 in f16 leaves sc*q exactly. (The bits of sc*q alone would
// be the f16 subnormal sc*q*2^-24, but the matrix cores round products of
// subnormal f16 operands more coarsely: about 4e-6 of the dot's magnitude
// against 2e-7 for normal operands, measured.)
__device__ __forceinline__ uint32_t scaled_u16(uint32_t p, uint32_t sc2) {
  const u16x2 m = __builtin_bit_cast(u16x2, p) * __builtin_bit_cast(u16x2, sc2) + (u16x2){0x6400, 0x6400};
  const f16x2 f = __builtin_bit_cast(f16x2, m) - (f16x2){(_Float16)1024.f, (_Float16)1024.f};
  return __builtin_bit_cast(uint32_t, f);
}
// Bytes 2H, 2H+1 of v (each below 16) times sch (two f16 copies of a 6-bit
// scale) as two exact normal f16 values sc*q, in two instructions: a byte
// below 16 read as FP8 E4M3 is q * 2^-9 exactly, v_cvt_scalef32_pk_f16_fp8
// scales it by 2^9 (the instruction takes only the exponent of its scale
// operand, so the scale must be a power of two) and q * sc <= 945 is an
// integer, exact in f16.
template <bool H>
__device__ __forceinline__ uint32_t nib_pair_sc(uint32_t v, f16x2 sch) {
  const f16x2 q = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 512.f, H);
  return __builtin_bit_cast(uint32_t, q * sch);
}
__device__ __forceinline__ f16x2 f16_pair(uint32_t sc) {
  const _Float16 h = (_Float16)(float)sc;
  return (f16x2){h, h};
}
// Word w of a gate/up lane chunk (positions 8v..8v+3 in the low nibbles,
// 8v+4..8v+7 in the high ones) times the scale sc, as 8 f16 values sc*q in
// position order.
__device__ __forceinline__ f16x8 burst_a(uint32_t w, uint32_t sc) {
  const uint32_t lo = nib_lo(w), hi = nib_hi(w);
  const f16x2 sch = f16_pair(sc);
  const u32x4 a = {nib_pair_sc<false>(lo, sch), nib_pair_sc<true>(lo, sch), nib_pair_sc<false>(hi, sch),
                   nib_pair_sc<true>(hi, sch)};
  return __builtin_bit_cast(f16x8, a);
}
// v split into the f16 part of the lane's column: hi = f16(v), lo = f16(v - hi).
__device__ __forceinline__ _Float16 f16_part(float v, bool lo) {
  const _Float16 h = (_Float16)v;
  return lo ? (_Float16)(v - (float)h) : h;
}
// Lane mq's dword v of its quad, masked to the two nibbles at bit `shift`
// and 16 + shift (the mask goes with the DPP read, so the move folds into
// the AND as its source modifier: the callers keep the mask opaque so that
// the compiler does not shift first), then shifted down: one output's two
// neurons as a u16 pair.
template <int MQ>
__device__ __forceinline__ uint32_t quad_nibbles(uint32_t v, uint32_t mask, uint32_t shift) {
  constexpr int ctrl = MQ | MQ << 2 | MQ << 4 | MQ << 6;
  return ((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xf, 0xf, true) & mask) >> shift;
}
// One down tile (outputs 16m..16m+15 of a super-block) for every column: A
// = sc*q of the lane's output (position q of the quad's unit) and neurons
// 8kg..8kg+7, the product started at the sub-block's min terms.
template <int MQ>
__device__ __forceinline__ f32x4 burst_tile(const uint4& U, uint32_t mask, uint32_t shift, const uint4& scp,
                                            const f16x8& bd, const f32x4& cmin) {
  const u32x4 a = {scaled_u16(quad_nibbles<MQ>(U.x, mask, shift), scp.x),
                   scaled_u16(quad_nibbles<MQ>(U.y, mask, shift), scp.y),
                   scaled_u16(quad_nibbles<MQ>(U.z, mask, shift), scp.z),
                   scaled_u16(quad_nibbles<MQ>(U.w, mask, shift), scp.w)};
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), bd, cmin, 0, 0, 0);
}
// Max over the 32 lanes of each half wavefront (quad butterflies, two row
// rotations, then the other row of the half through a swizzle).
__device__ __forceinline__ float half_wave_max(float m) {
  m = fmaxf(m, dpp_f<kQuadXor1>(m));
  m = fmaxf(m, dpp_f<kQuadXor2>(m));
  m = fmaxf(m, dpp_f<kRowRor4>(m));
  m = fmaxf(m, dpp_f<kRowRor8>(m));
  return fmaxf(m, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(m), 0x401F)));   // lane ^ 16
}

__global__ __launch_bounds__(kDecodeThreads) void decode_burst_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  const PlanHeader* PH = reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + plan_field(PH, offsetof(PlanHeader, pairs_off)));
  const unsigned hidden = plan_field(PH, offsetof(PlanHeader, hidden)), nsb = hidden / 256;
  const unsigned np = plan_field(PH, offsetof(PlanHeader, npairs)), tpw = plan_field(PH, offsetof(PlanHeader, tpw));
  const unsigned burst = plan_field(PH, offsetof(PlanHeader, burst));
  // Each pair's partial index for tokens 0..7 (after the token table).
  const uint32_t* bpart = reinterpret_cast<const uint32_t*>(plan + plan_field(PH, offsetof(PlanHeader, groups_off)) +
                                                          burst * sizeof(DecodeToken));
  const float* xg = reinterpret_cast<const float*>(plan + plan_field(PH, offsetof(PlanHeader, x_off)));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) BurstShared SH;
  BurstLds& L = SH.pair;
  const unsigned kg = (unsigned)lane >> 4, col = (unsigned)lane & 15, tok = col >> 1;
  const bool lo_part = (col & 1) != 0, tin = tok < burst;
  const unsigned sb0 = 2 * (unsigned)wave, sb1 = sb0 + 1;
  const bool has0 = sb0 < nsb, has1 = sb1 < nsb;
  const unsigned lb0 = min(sb0, nsb - 1), lb1 = min(sb1, nsb - 1);
  // Down offsets: lane 16kg + 4a + q loads unit (kg, 4(4G + q) + a); the
  // header of neuron l%32 of super-block 2w + l/32.
  const unsigned qa = ((unsigned)lane >> 2) & 3, qq = (unsigned)lane & 3;
  const uint32_t voff_u = 1024 * kg + 64 * qq + 16 * qa;
  const uint32_t voff_h = 4608 * ((unsigned)lane >> 5 ? lb1 : lb0) + 16 * ((unsigned)lane & 31);
  const bool dh_valid = 2 * (unsigned)wave + ((unsigned)lane >> 5) < nsb;
  uint32_t bad = 0;

  unsigned p = blockIdx.x * tpw;   // this workgroup's chunk: pairs [p, min(p + tpw, np))
  const unsigned pend = min(p + tpw, np);
  PairBuf B = pair_buf(pairs + p);

  // x of the burst into B operands: lane (kg, column) of wavefront w holds,
  // for super-block 2w + s, sub-blocks kg and 4 + kg of the column's token
  // (its hi or lo part), for all of the workgroup's pairs. The workgroup
  // stages up to 4 tokens at a time in LDS: thread i takes values
  // 8i..8i+7 of each token (the 32 threads of a super-block agree on its
  // power of two), then every lane reads its operands. The first chunk's x
  // is requested before the first pair's bytes, so that waiting for it does
  // not wait for the weights.
  const unsigned v0 = 8 * (unsigned)tid, sbx = (unsigned)tid >> 5;
  const bool xlive = v0 < hidden;
  float4 xv[kStageTokens][2];
  auto load_x = [&](unsigned c0) {
    const unsigned nt = min(burst - c0, (unsigned)kStageTokens);
#pragma unroll
    for (unsigned tl = 0; tl < (unsigned)kStageTokens; ++tl) {
      const float* xt = xg + (size_t)(c0 + min(tl, nt - 1)) * hidden + (xlive ? v0 : 0);
      xv[tl][0] = *reinterpret_cast<const float4*>(xt);
      xv[tl][1] = *reinterpret_cast<const float4*>(xt + 4);
    }
  };
  load_x(0);
  BurstRound R[4];
  BurstHdr HD;
  load_burst_hdr(B, lb0, lb1, lane, HD);
  load_burst_round(B, 0, lb0, lb1, lane, R[0]);
  load_burst_round(B, 1, lb0, lb1, lane, R[1]);
  __builtin_amdgcn_sched_barrier(0);

  f16x8 bx[2][2][4];   // [super-block][part p][word v]: positions 8v..8v+7 of sub-block 4p + kg
  float xsm[2][2];     // sum of x over sub-block 4p + kg (hi columns of the burst's tokens; 0 otherwise)
  int xe[2];           // e of the column's token in the super-block
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    xe[s] = 0;
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      xsm[s][pp] = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) bx[s][pp][v] = f16x8{};
    }
  }
  {
    BurstStage& X = SH.stage;
    for (unsigned c0 = 0; c0 < burst; c0 += kStageTokens) {
      const unsigned nt = min(burst - c0, (unsigned)kStageTokens);
      if (c0) {
        load_x(c0);
        __syncthreads();   // the previous chunk's operands are read
      }
#pragma unroll
      for (unsigned tl = 0; tl < (unsigned)kStageTokens; ++tl) {
        const float v8[8] = {xv[tl][0].x, xv[tl][0].y, xv[tl][0].z, xv[tl][0].w,
                             xv[tl][1].x, xv[tl][1].y, xv[tl][1].z, xv[tl][1].w};
        float m = 0.f, sum = 0.f;
        bool fin = true;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          m = fmaxf(m, fabsf(v8[k]));
          fin = fin && isfinite(v8[k]);
          sum += v8[k];
        }
        if (!fin && xlive && tl < nt) bad |= kErrRange;   // a non-finite x makes the token's a non-finite
        m = half_wave_max(m);
        sum += dpp_f<kQuadXor1>(sum);
        sum += dpp_f<kQuadXor2>(sum);   // the 4 threads of a 32-value sub-block
        int E = 0;
        if (m > 0.f) (void)frexpf(m, &E);   // m < 2^E over the super-block
        const int e = E - 15;
        f16x8 hi, lo;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float xp = fin ? ldexpf(v8[k], -e) : 0.f;
          hi[k] = (_Float16)xp;
          lo[k] = (_Float16)(xp - (float)hi[k]);
        }
        if (xlive) {
          *reinterpret_cast<f16x8*>(&X.x[2 * tl][v0]) = hi;
          *reinterpret_cast<f16x8*>(&X.x[2 * tl + 1][v0]) = lo;
          if ((tid & 3) == 0) X.sum[tl][v0 / 32] = fin ? sum : 0.f;
          if ((tid & 31) == 0) X.e[tl][sbx] = e;
        }
      }
      __syncthreads();   // the chunk is in LDS
      // Lanes whose token is in this chunk take their operands.
      const bool mine = tin && tok >= c0 && tok < c0 + nt;
      const unsigned row = 2 * min(tok - min(tok, c0), (unsigned)kStageTokens - 1) + (lo_part ? 1u : 0u);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const unsigned sb = s ? lb1 : lb0;
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            // Columns of tokens past the burst take a staged token's values:
            // their products are never used.
            const f16x8 r = *reinterpret_cast<const f16x8*>(&X.x[row][256 * sb + 32 * (4 * pp + kg) + 8 * v]);
            bx[s][pp][v] = mine || c0 == 0 ? r : bx[s][pp][v];
          }
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const float sm = X.sum[row >> 1][8 * sb + 4 * pp + kg];
          xsm[s][pp] = mine && !lo_part ? sm : xsm[s][pp];
        }
        const int e = X.e[row >> 1][sb];
        xe[s] = mine ? e : xe[s];
      }
    }
    __syncthreads();   // the staging area becomes the pair loop's
  }

  float* rowp_w = &L.rowp[0][wave][tok][4 * kg];
  for (;;) {
    const unsigned q = p + 1;
    const bool more = q < pend;
    const PairBuf Bn = pair_buf(pairs + (more ? q : p), more);
    const uint32_t tmask = uniform(plan_read(reinterpret_cast<const uint32_t*>(pairs + p) + 3)) >> 16 & 0xffu;
    float gate = 0.f;   // the column's token's gate (scalar reads, then a per-lane pick)
    uint32_t units[kMaxBurst];   // each token's partial index
    {
      const uint32_t* gw = reinterpret_cast<const uint32_t*>(pairs[p].gate);
#pragma unroll
      for (unsigned t = 0; t < (unsigned)kMaxBurst; ++t) {
        const float g = __uint_as_float(uniform(plan_read(gw + t)));
        units[t] = uniform(plan_read(bpart + (size_t)p * kMaxBurst + t));
        gate = tok == t ? g : gate;
      }
    }
    // The pair's gate/up headers into this wavefront's LDS, with each d.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      L.hdr[wave][s][lane] = HD.h[s];
      L.dg[wave][s][lane] = half_to_float(HD.h[s].x & 0xffff);
    }
    __builtin_amdgcn_wave_barrier();
    BurstDown D;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      __builtin_amdgcn_sched_barrier(0);
      // Two rounds ahead: rounds 2 and 3, the down, then the next pair's
      // headers and rounds 0 and 1 (zeros after the last pair).
      if (rb < 2) load_burst_round(B, rb + 2, lb0, lb1, lane, R[rb + 2]);
      if (rb == 1) load_burst_down(B, lb0, lb1, voff_u, voff_h, D);
      if (rb == 2) {
        load_burst_hdr(Bn, lb0, lb1, lane, HD);
        load_burst_round(Bn, 0, lb0, lb1, lane, R[0]);
      }
      if (rb == 3) load_burst_round(Bn, 1, lb0, lb1, lane, R[1]);
      __builtin_amdgcn_sched_barrier(0);
      const BurstRound& C = R[rb];
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      f32x4 cmin = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (!(s ? has1 : has0)) continue;
        const uint4 hc = L.hdr[wave][s][16 * rb + col];   // row i = col of this row-block
        const float4 drow = *reinterpret_cast<const float4*>(&L.dg[wave][s][16 * rb + 4 * kg]);
        if (half_bad(hc.x) || half_bad(hc.x >> 16)) bad |= kErrScale;
        const float dmn = half_to_float(hc.x >> 16);
        uint32_t sc0, mi0, sc1, mi1;
        q4k_scale_min(hc.y, hc.z, hc.w, kg, sc0, mi0);
        q4k_scale_min(hc.y, hc.z, hc.w, 4 + kg, sc1, mi1);
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < 4; ++v)
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(burst_a(word(C.q[s][0], v), sc0), bx[s][0][v], c, 0,
                                                     0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(burst_a(word(C.q[s][1], v), sc1), bx[s][1][v], c, 0,
                                                     0, 0);
        cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(-dmn * (float)mi0, xsm[s][0], cmin, 0, 0, 0);
        cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(-dmn * (float)mi1, xsm[s][1], cmin, 0, 0, 0);
        acc[0] = fmaf(c[0], ldexpf(drow.x, xe[s]), acc[0]);
        acc[1] = fmaf(c[1], ldexpf(drow.y, xe[s]), acc[1]);
        acc[2] = fmaf(c[2], ldexpf(drow.z, xe[s]), acc[2]);
        acc[3] = fmaf(c[3], ldexpf(drow.w, xe[s]), acc[3]);
      }
      float v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v4[r] = acc[r] + cmin[r];
        v4[r] += dpp_f<kQuadXor1>(v4[r]);   // hi + lo of the column pair
      }
      if (!lo_part) *reinterpret_cast<float4*>(rowp_w + rb * (kDecodeWaves * kMaxBurst * 20)) =
          make_float4(v4[0], v4[1], v4[2], v4[3]);
      __syncthreads();   // every wavefront's row sums of row-block rb are in LDS
      if (wave == rb) {
        // Lane (neuron i, token t): a = gate row i, u = up row 8 + i.
        const unsigned i = (unsigned)lane >> 3, t = (unsigned)lane & 7;
        float a = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
          a += L.rowp[rb][w][t][i];
          u += L.rowp[rb][w][t][8 + i];
        }
        const float g = __shfl(gate, (int)(2 * t));
        float hv = 0.f;
        if (t < burst && (tmask >> t & 1u)) {
          uint32_t hb = 0;
          hv = g * silu_mul_f32(a, u, hb);
          bad |= hb;
        }
        L.h[t][8 * rb + i] = hv;
      }
    }
    __syncthreads();   // the pair's h is in LDS

    // Down tables from the neuron headers (this wavefront's own LDS).
    {
      const uint4 dh = D.h;
      const unsigned n = (unsigned)lane & 31, s = (unsigned)lane >> 5;
      if (dh_valid && (half_bad(dh.x) || half_bad(dh.x >> 16))) bad |= kErrScale;
      L.dd[wave][s][n] = half_to_float(dh.x & 0xffff);
      L.dm[wave][s][n] = half_to_float(dh.x >> 16);
      const uint32_t sc_lo = dh.y & 0x3F3F3F3Fu, mi_lo = dh.z & 0x3F3F3F3Fu;
      const uint32_t sc_hi = (dh.w & 0x0F0F0F0Fu) | ((dh.y >> 2) & 0x30303030u);
      const uint32_t mi_hi = ((dh.w >> 4) & 0x0F0F0F0Fu) | ((dh.z >> 2) & 0x30303030u);
      uint16_t* ts = reinterpret_cast<uint16_t*>(&L.dsc[wave][s][0][0]);
      uint16_t* tm = reinterpret_cast<uint16_t*>(&L.dmn[wave][s][0][0]);
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        ts[32 * g + n] = (uint16_t)((g < 4 ? sc_lo : sc_hi) >> (8 * (g & 3)) & 0xffu);
        const float mf = (float)((g < 4 ? mi_lo : mi_hi) >> (8 * (g & 3)) & 0xffu);
        tm[32 * g + n] = __builtin_bit_cast(uint16_t, (_Float16)mf);   // m as an f16 operand
      }
    }
    __builtin_amdgcn_wave_barrier();
    {
      // B of the down: d*gate*h and -dmin*gate*h of neurons 8kg..8kg+7 for
      // the column's token, over a power of two per (super-block, token).
      const float4 ha = *reinterpret_cast<const float4*>(&L.h[tok][8 * kg]);
      const float4 hb4 = *reinterpret_cast<const float4*>(&L.h[tok][8 * kg + 4]);
      const float hv[8] = {ha.x, ha.y, ha.z, ha.w, hb4.x, hb4.y, hb4.z, hb4.w};
      const uint32_t shift = 4 * qq;
      uint32_t mask = 0x000F000Fu << shift;
      asm volatile("" : "+v"(mask));   // kept as (x & mask) >> shift: the AND takes the DPP read
      float* outw = &L.out[wave][tok][4 * kg];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (!(s ? has1 : has0)) continue;
        float cd[8], cm[8], m = 0.f;
        {
          const float4 d0 = *reinterpret_cast<const float4*>(&L.dd[wave][s][8 * kg]);
          const float4 d1 = *reinterpret_cast<const float4*>(&L.dd[wave][s][8 * kg + 4]);
          const float4 m0 = *reinterpret_cast<const float4*>(&L.dm[wave][s][8 * kg]);
          const float4 m1 = *reinterpret_cast<const float4*>(&L.dm[wave][s][8 * kg + 4]);
          const float dv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
          const float mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            cd[j] = dv[j] * hv[j];
            cm[j] = -mv[j] * hv[j];
            m = fmaxf(m, fmaxf(fabsf(cd[j]), fabsf(cm[j])));
          }
        }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        int E = 0;
        if (m > 0.f) (void)frexpf(m, &E);
        const int e = E - 15;
        f16x8 bd, bm;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          bd[j] = f16_part(ldexpf(cd[j], -e), lo_part);
          bm[j] = f16_part(ldexpf(cm[j], -e), lo_part);
        }
        const int ye = e;
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int G = 0; G < 4; ++G) {
          // Tiles 4G..4G+3: sub-blocks 2G (tiles 4G, 4G+1) and 2G+1.
          const uint4 sc0 = L.dsc[wave][s][2 * G][kg], sc1 = L.dsc[wave][s][2 * G + 1][kg];
          const f32x4 cm0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(f16x8, L.dmn[wave][s][2 * G][kg]), bm, z, 0, 0, 0);
          const f32x4 cm1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(f16x8, L.dmn[wave][s][2 * G + 1][kg]), bm, z, 0, 0, 0);
          const uint4 U = D.u[s][G];
          f32x4 c[4];
          c[0] = burst_tile<0>(U, mask, shift, sc0, bd, cm0);
          c[1] = burst_tile<1>(U, mask, shift, sc0, bd, cm0);
          c[2] = burst_tile<2>(U, mask, shift, sc1, bd, cm1);
          c[3] = burst_tile<3>(U, mask, shift, sc1, bd, cm1);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // Outputs 16(4G + k) + 4kg..+3 of the column: hi + lo (the
            // store below applies 2^ye).
            float4 y4;
            y4.x = c[k][0] + dpp_f<kQuadXor1>(c[k][0]);
            y4.y = c[k][1] + dpp_f<kQuadXor1>(c[k][1]);
            y4.z = c[k][2] + dpp_f<kQuadXor1>(c[k][2]);
            y4.w = c[k][3] + dpp_f<kQuadXor1>(c[k][3]);
            if (!lo_part) *reinterpret_cast<float4*>(outw + 16 * (4 * G + k)) = y4;
          }
        }
        __builtin_amdgcn_wave_barrier();
        // The super-block's outputs of each routed token, times 2^ye,
        // stored whole: lane l takes outputs 4l..4l+3, positions 512w +
        // 256(l%2) + 4(32s + l/2) of decode_kernel's layout.
        const unsigned pos = 512 * (unsigned)wave + 256 * ((unsigned)lane & 1) + 4 * (32 * (unsigned)s + ((unsigned)lane >> 1));
        for (uint32_t tm = tmask; tm; tm &= tm - 1) {
          const unsigned t = (unsigned)__builtin_ctz(tm);
          uint32_t unit = units[0];
#pragma unroll
          for (unsigned k = 1; k < (unsigned)kMaxBurst; ++k) unit = t == k ? units[k] : unit;
          const int yt = __builtin_amdgcn_readlane(ye, (int)(2 * t));   // the token's hi column
          const float4 y4 = *reinterpret_cast<const float4*>(&L.out[wave][t][4 * lane]);
          *reinterpret_cast<float4*>(S.wgpart + partial_index(unit, pos, S.ustride)) =
              make_float4(ldexpf(y4.x, yt), ldexpf(y4.y, yt), ldexpf(y4.z, yt), ldexpf(y4.w, yt));
        }
        __builtin_amdgcn_wave_barrier();   // the outputs are read before the next super-block writes them
      }
    }
    if (!more) break;
    p = q;
    B = Bn;
  }
  if (bad) flag(status, bad);
}

// ------------------------------------------------- decode kernel, ref-q8
//
// The ref-q8 arithmetic (backends/ref.c:66,85: x quantized per 64 and h per
// 32 by fr_q8_activation, src/q4.c:37-61; dots, SiLU and the gated sum in
// double) on decode_kernel's work list and tiles: Q4_K gate/up with the
// transposed Q4_K down, T <= 8.
//
// A quantized value is q = (float)(k*s), k an integer in [-127, 127] and s
// the group's scale. k*s needs up to 31 bits, but its rounding error is a
// multiple of u = 2^(floor(log2 s) - 23) (the last bit of s; 2^-149 for a
// subnormal s) of at most 64u, so q = s*k + u*r exactly with k and r signed
// bytes. x is staged as these two digits, and the same int8 matrix products
// as decode_kernel's give exact integer dots of each row with k and with r
// per 32-value sub-block. Everything after them is double: each dot times
// d*sc times its digit's weight is exact before the sum, the min term uses
// the exact sum of the sub-block's values, so a and u differ from the
// reference's double dots only in the order of the additions. That holds
// where the reference's float weight (d*sc)*q - dmin*mi (src/native.c:14-22)
// is exact, which is the case when the fp16 exponents of d and dmin differ
// by -7..3; a super-block header outside that range sets kErrInexact, and
// fr_hip_run then runs the request on layer_kernel, which decodes every
// weight as the reference does.
//
// h = SiLU(a)*u as in ref (a and u narrowed to float, the sigmoid in
// double), quantized per 32 (the unit's 32 neurons), so the down follows
// the fourth round: the four rounds' down bytes stay in registers, and the
// down is double FMAs over the nibbles (as q*2^-9 from the FP8 conversion,
// exact). The unit's partial gate*dot is stored in double; decode_reduce
// sums a token's partials in double in the reference's order.
constexpr uint32_t kErrInexact = 8;   // a weight the reference rounds in float (ref-q8 decode only)

struct DecodeQ8Table {                 // one wavefront's down coefficients of one round
  double D[2][8][8];                   // [super-block][group][neuron] d*sc*h
  double M[2][8][8];                   // dmin*mi*h
};
struct DecodeQ8Lds {
  int8_t xd[2][4][kSubBlocks][32];     // [x slot][digit][sub-block][value]: k, r, 0, 0
  float xw[2][kSubBlocks][4];          // [x slot][sub-block][digit]: s, u, 0, 0
  double xs[2][kSubBlocks];            // exact sum of each sub-block's quantized values
  float dsc[kDecodeWaves][16][64];     // [wave][sub-block of its super-blocks][row] d*sc
  double rowp[2][kDecodeWaves][64];    // [unit parity][wave][row] scaled integer dots
  double minp[2][kDecodeWaves][64];    // [unit parity][wave][row] min terms
  float h[kDecodeWaves][32];           // the unit's h, then quantized (each wavefront's own copy)
  uint4 dh[kDecodeWaves][16];
  DecodeQ8Table table[kDecodeWaves];
};
static_assert(sizeof(DecodeQ8Lds) <= 160 * 1024, "ref-q8 decode LDS");

// The reference's float weight is exact for every scale, min and quant of a
// header whose d and dmin exponents differ by -7..3 (either one zero is exact
// too); subnormals count as exponent -14.
__device__ __forceinline__ bool q4k_weights_exact(uint32_t dm) {
  const int ed = max((int)((dm >> 10) & 31u), 1), em = max((int)((dm >> 26) & 31u), 1);
  const bool zero = (dm & 0x7fffu) == 0 || (dm & 0x7fff0000u) == 0;
  return zero || (ed - em <= 3 && em - ed <= 7);
}

// fr_q8_activation of x (src/q4.c:37-61) and its two-digit staging: thread
// t holds values 8(t%4)..+7 of sub-block t/4; the eight threads of a 64-value
// group agree on its largest magnitude.
// With kLanes the digits go to the row-format kernel's lane-major layout
// (as stage_x's), each sub-block's weights and exact sum to its tables.
template <class Lds, bool kLanes = false>
__device__ __forceinline__ void stage_x_q8(const float4 (&v4)[2], unsigned slot, unsigned nsub, Lds& L,
                                           uint32_t& bad) {
  const unsigned tid = threadIdx.x, s = tid >> 2, q = tid & 3;
  const float v[8] = {v4[0].x, v4[0].y, v4[0].z, v4[0].w, v4[1].x, v4[1].y, v4[1].z, v4[1].w};
  float m = 0.f;
  uint32_t fin = 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m = fmaxf(m, fabsf(v[i]));
    fin &= isfinite(v[i]) ? 1u : 0u;
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    m = fmaxf(m, __shfl_xor(m, o));
    fin &= (uint32_t)__shfl_xor((int)fin, o);
  }
  if (!fin && s < nsub) bad |= kErrRange;   // fr_q8_activation's FR_NUMERIC
  const float scale = m / 127.0f, inv = 127.0f / m;
  const bool zero = scale == 0.f || !fin, finite_inv = isfinite(inv);
  int es = 0;
  (void)frexpf(scale, &es);                 // scale in [2^(es-1), 2^es)
  const int ue = max(es - 24, -149);
  const double ud = ldexp(1.0, ue);
  uint32_t w[2][2] = {{0u, 0u}, {0u, 0u}};
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float r = finite_inv ? v[i] * inv : (v[i] / m) * 127.0f;
    r = fminf(fmaxf(rintf(r), -127.f), 127.f);
    const double back = fmin(fmax((double)r * (double)scale, -(double)FLT_MAX), (double)FLT_MAX);
    const float xq = zero ? 0.f : (float)back;
    const int k = zero ? 0 : (int)r;
    const int rem = (int)(((double)xq - (double)k * (double)scale) / ud);   // exact: a multiple of u
    if (rem < -127 || rem > 127) bad |= kErrRange;                          // only where k*s passes FLT_MAX
    w[0][i >> 2] |= (uint32_t)(k & 255) << (8 * (i & 3));
    w[1][i >> 2] |= (uint32_t)(rem & 255) << (8 * (i & 3));
    sum += (double)xq;                      // exact: multiples of u below 2^37 u
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  if (s < nsub) {
    const float ws = zero ? 0.f : scale, wu = zero ? 0.f : (float)ud;
    if constexpr (kLanes) {
#pragma unroll
      for (int d = 0; d < 2; ++d)
        *reinterpret_cast<uint2*>(&L.xl[d][s & 1][q >> 1][s >> 1][2 * (q & 1)]) = make_uint2(w[d][0], w[d][1]);
      if (q == 0) {
        *reinterpret_cast<float2*>(&L.xw[s][0]) = make_float2(ws, wu);
        L.xsd[s] = sum;
      }
    } else {
      *reinterpret_cast<uint2*>(&L.xd[slot][0][s][8 * q]) = make_uint2(w[0][0], w[0][1]);
      *reinterpret_cast<uint2*>(&L.xd[slot][1][s][8 * q]) = make_uint2(w[1][0], w[1][1]);
      *reinterpret_cast<uint2*>(&L.xd[slot][2][s][8 * q]) = make_uint2(0u, 0u);
      *reinterpret_cast<uint2*>(&L.xd[slot][3][s][8 * q]) = make_uint2(0u, 0u);
      if (q == 0) {
        *reinterpret_cast<float4*>(&L.xw[slot][s][0]) = make_float4(ws, wu, 0.f, 0.f);
        L.xs[slot][s] = sum;
      }
    }
  }
}

// ------------------------------------------------- q8_256: the AVX2 arithmetic
//
// The AVX2 backend's native path quantizes x once per token with quantize8
// (backends/avx2.c:184-203, group 256 at :633): d = amax/127, inv = amax ?
// 127/amax : 0, codes by the cvtps conversion of x*inv (round to nearest
// even; NaN and values outside int32 give INT32_MIN), saturated through
// int16 to int8, and an int16 sum per 32 of the unsaturated codes (wrapping).
// Its dots are integer (codes times the 6-bit scales or int8 weights) times
// one float scale per block, h is SiLU in float (:428) quantized per 32 by
// the same routine (:434), and the down is integer (codes times h codes)
// times the block scale, md and the gate (:331-362, :364-390).

// cvtps of one float (backends/avx2.c:193-196).
__device__ __forceinline__ int cvtps_i32(float r) {
  return (r != r || !(fabsf(r) < 2147483648.f)) ? INT_MIN : (int)rintf(r);
}
// The int8 code of a cvtps result: int32 -> int16 -> int8, saturating.
__device__ __forceinline__ int sat_i8(int v) { return min(max(v, -128), 127); }

// quantize8 of x per 256 in the row-format kernel's lane-major layout
// (digit 0 the code; the q8_256 dots read no other): thread t holds values 8(t%4)..+7 of
// sub-block t/4; the 32 threads of a 256-group agree on its largest
// magnitude. Each sub-block's weight is the group's d, its sum the int16 sum
// of its codes times d (exact in double).
template <class Lds>
__device__ __forceinline__ void stage_x_q256(const float4 (&v4)[2], unsigned nsub, Lds& L, uint32_t& bad) {
  const unsigned tid = threadIdx.x, s = tid >> 2, q = tid & 3;
  const float v[8] = {v4[0].x, v4[0].y, v4[0].z, v4[0].w, v4[1].x, v4[1].y, v4[1].z, v4[1].w};
  float m = 0.f;
  uint32_t fin = 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m = fmaxf(m, fabsf(v[i]));
    fin &= isfinite(v[i]) ? 1u : 0u;
  }
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
    m = fmaxf(m, __shfl_xor(m, o));
    fin &= (uint32_t)__shfl_xor((int)fin, o);
  }
  if (!fin && s < nsub) bad |= kErrRange;   // the reference's run rejects a non-finite x first (backends/avx2.c:626)
  const float d = m / 127.0f, inv = m != 0.f ? 127.0f / m : 0.f;
  uint32_t w[2] = {0u, 0u}, sum = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = cvtps_i32(v[i] * inv);
    sum += (uint32_t)c;
    w[i >> 2] |= (uint32_t)(sat_i8(c) & 255) << (8 * (i & 3));
  }
  sum += (uint32_t)__shfl_xor((int)sum, 1);
  sum += (uint32_t)__shfl_xor((int)sum, 2);
  if (s < nsub) {
    *reinterpret_cast<uint2*>(&L.xl[0][s & 1][q >> 1][s >> 1][2 * (q & 1)]) = make_uint2(w[0], w[1]);
    if (q == 0) {
      *reinterpret_cast<float2*>(&L.xw[s][0]) = make_float2(d, 0.f);
      L.xsd[s] = (double)(int16_t)(uint16_t)sum * (double)d;
    }
  }
}

// quantize8 of the unit's 32 h (group 32, no sums), held by lanes 0..31 of
// the wavefront: h[n] becomes its code, *md the group's d.
__device__ __forceinline__ void quantize_h32_q256(float* h, float* md, int lane) {
  const float v = lane < 32 ? h[lane] : 0.f;
  float m = fabsf(v);
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float inv = m != 0.f ? 127.0f / m : 0.f;
  const float code = (float)sat_i8(cvtps_i32(v * inv));
  __builtin_amdgcn_wave_barrier();
  if (lane < 32) h[lane] = code;
  if (lane == 0) *md = m / 127.0f;
  __builtin_amdgcn_wave_barrier();
}

// SiLU(a)*u as the AVX2 native path forms it, a/(1+e^-a)*u in float
// (backends/avx2.c:428); a non-finite h is its FR_NUMERIC (:433).
__device__ __forceinline__ float silu_mul_q256(float a, float u, uint32_t& bad) {
  const float h = a / (1.f + expf(-a)) * u;
  if (!isfinite(h)) {
    bad |= kErrRange;
    return 0.f;
  }
  return h;
}

// Headers of super-block sb into the d*sc table (as decode_kernel's header
// pass); the min term over the super-block in double, exact per sub-block.
__device__ __forceinline__ double header_pass_q8(const uint4& h, unsigned sb, unsigned sbl, unsigned t, int wave,
                                                 int lane, DecodeQ8Lds& L, uint32_t& bad) {
  if (half_bad(h.x) || half_bad(h.x >> 16)) bad |= kErrScale;
  if (!q4k_weights_exact(h.x)) bad |= kErrInexact;
  const float d = half_to_float(h.x & 0xffff), dm = half_to_float(h.x >> 16);
  const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, mi_lo = h.z & 0x3F3F3F3Fu;
  const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
  const uint32_t mi_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  double mins = 0.0;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const float sc = ub(g < 4 ? sc_lo : sc_hi, g & 3), mi = ub(g < 4 ? mi_lo : mi_hi, g & 3);
    L.dsc[wave][8 * sbl + g][lane] = d * sc;
    mins += (double)(dm * mi) * L.xs[t][8 * sb + g];
  }
  return mins;
}

// x operands as decode_kernel's (digits 2 and 3 are zero), each column's
// weight from the staged table.
__device__ __forceinline__ void x_operands_q8(unsigned t, unsigned sb, int lane, const DecodeQ8Lds& L, i32x4 (&b)[4],
                                              double (&fx)[2]) {
  const unsigned kg = (unsigned)lane >> 4, j = (unsigned)lane & 15, js = j >> 2, jd = j & 3;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned G = (unsigned)m >> 1, hh = (unsigned)m & 1;
    const i32x4 z = {0, 0, 0, 0};
    b[m] = js == kg ? *reinterpret_cast<const i32x4*>(&L.xd[t][jd][8 * sb + 4 * G + kg][16 * hh]) : z;
  }
#pragma unroll
  for (int G = 0; G < 2; ++G) fx[G] = (double)L.xw[t][8 * sb + 4 * G + js][jd];
}

__device__ __forceinline__ void rb_products_q8(const uint4 (&q)[2], const i32x4 (&b)[4], const double (&fx)[2],
                                               unsigned sbl, unsigned rb, int wave, int lane, const DecodeQ8Lds& L,
                                               double (&acc)[4]) {
  const unsigned kg = (unsigned)lane >> 4, js = ((unsigned)lane & 15) >> 2;
#pragma unroll
  for (int G = 0; G < 2; ++G) {
    const uint4 w = q[G];
    i32x4 c = {0, 0, 0, 0};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint32_t w0 = hh ? w.z : w.x, w1 = hh ? w.w : w.y;
      const i32x4 a = {(int)nib_lo(w0), (int)nib_hi(w0), (int)nib_lo(w1), (int)nib_hi(w1)};
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[2 * G + hh], c, 0, 0, 0);
    }
    const float4 ds = *reinterpret_cast<const float4*>(&L.dsc[wave][8 * sbl + 4 * G + js][16 * rb + 4 * kg]);
    acc[0] = fma((double)c[0], (double)ds.x * fx[G], acc[0]);
    acc[1] = fma((double)c[1], (double)ds.y * fx[G], acc[1]);
    acc[2] = fma((double)c[2], (double)ds.z * fx[G], acc[2]);
    acc[3] = fma((double)c[3], (double)ds.w * fx[G], acc[3]);
  }
}

__device__ __forceinline__ double row_sum_d(double v) {
  v += dpp_d<kQuadXor1>(v);
  v += dpp_d<kQuadXor2>(v);
  v += dpp_d<kRowRor4>(v);
  v += dpp_d<kRowRor8>(v);
  return v;
}

// Down projection of round r (neurons 8r..8r+7, quantized h in hs[0..7]) in
// double: coefficients, then 8 outputs per lane added into y.
__device__ __forceinline__ void down_round_q8(const DecodeDnBytes& R, const float* hs, int wave, int lane,
                                              unsigned nsb, DecodeQ8Lds& L, double (&y)[8], uint32_t& bad) {
  if (lane < 16) L.dh[wave][lane] = R.dh;
  DecodeQ8Table& T = L.table[wave];
  {
    const unsigned ts = (unsigned)lane >> 5, tg = ((unsigned)lane >> 2) & 7, n0 = 2 * ((unsigned)lane & 3);
    const bool tvalid = 2 * (unsigned)wave + ts < nsb;
    double Dv[2], Mv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4 hdr = L.dh[wave][8 * ts + n0 + q];
      bool ok;
      float D, M;
      hdr_dm(hdr, tg, D, M, ok);
      if (tvalid && !ok) bad |= kErrScale;
      if (tvalid && !q4k_weights_exact(hdr.x)) bad |= kErrInexact;
      const double hv = (double)hs[n0 + q];
      Dv[q] = (double)D * hv * (double)kFp8Nibble;   // exact: the nibbles below are q * 2^-9
      Mv[q] = (double)M * hv;
    }
    *reinterpret_cast<double2*>(&T.D[ts][tg][n0]) = make_double2(Dv[0], Dv[1]);
    *reinterpret_cast<double2*>(&T.M[ts][tg][n0]) = make_double2(Mv[0], Mv[1]);
  }
  __builtin_amdgcn_wave_barrier();
  const unsigned sbl = (unsigned)lane >> 5, j = (unsigned)lane & 31, g = j >> 2;
  if (2 * (unsigned)wave + sbl < nsb) {
    const double* cd = &T.D[sbl][g][0];
    const double* cm = &T.M[sbl][g][0];
    double coef[8], msum = 0.0;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      coef[n] = cd[n];
      msum += cm[n];
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint4 dq = R.dq[half];
      double s4[4] = {-msum, -msum, -msum, -msum};
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t v = word(dq, wd);
        const uint32_t lo = nib_lo(v), hi = nib_hi(v);
        const float2 la = nib_pair<false>(lo), lb = nib_pair<true>(lo), ha = nib_pair<false>(hi), hb = nib_pair<true>(hi);
        const double ca = coef[2 * wd], cb = coef[2 * wd + 1];
        s4[0] = fma((double)la.x, ca, s4[0]);
        s4[1] = fma((double)ha.x, ca, s4[1]);
        s4[2] = fma((double)la.y, ca, s4[2]);
        s4[3] = fma((double)ha.y, ca, s4[3]);
        s4[0] = fma((double)lb.x, cb, s4[0]);
        s4[1] = fma((double)hb.x, cb, s4[1]);
        s4[2] = fma((double)lb.y, cb, s4[2]);
        s4[3] = fma((double)hb.y, cb, s4[3]);
      }
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) y[4 * half + cc] += s4[cc];
    }
  }
  __builtin_amdgcn_wave_barrier();   // the table and headers are read before the next round writes them
}

// The unit's partial gate*dot in double, at decode_kernel's positions.
__device__ __forceinline__ void store_partial_q8(double* wgpart, unsigned stride, unsigned unit, int wave, int lane,
                                                 float gate, double (&y)[8]) {
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    double* p = wgpart + partial_index(unit, 4 * (128 * wave + 64 * hh + lane), stride);
    *reinterpret_cast<double2*>(p) = make_double2((double)gate * y[4 * hh], (double)gate * y[4 * hh + 1]);
    *reinterpret_cast<double2*>(p + 2) = make_double2((double)gate * y[4 * hh + 2], (double)gate * y[4 * hh + 3]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = 0.0;
}

// fr_q8_activation of the unit's 32 h, held by lanes 0..31 of every wavefront.
__device__ __forceinline__ void quantize_h32(float* h, int lane) {
  const float v = lane < 32 ? h[lane] : 0.f;
  float m = fabsf(v);
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float scale = m / 127.0f, inv = 127.0f / m;
  float r = isfinite(inv) ? v * inv : (v / m) * 127.0f;
  r = fminf(fmaxf(rintf(r), -127.f), 127.f);
  const double back = fmin(fmax((double)r * (double)scale, -(double)FLT_MAX), (double)FLT_MAX);
  const float hq = scale == 0.f ? 0.f : (float)back;
  __builtin_amdgcn_wave_barrier();
  if (lane < 32) h[lane] = hq;
  __builtin_amdgcn_wave_barrier();
}

__global__ __launch_bounds__(kDecodeThreads) void decode_q8_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  const PlanHeader* PH = reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + plan_field(PH, offsetof(PlanHeader, pairs_off)));
  const unsigned hidden = plan_field(PH, offsetof(PlanHeader, hidden)), nsb = hidden / 256, nsub = hidden / 32;
  const unsigned np = plan_field(PH, offsetof(PlanHeader, npairs)), tpw = plan_field(PH, offsetof(PlanHeader, tpw));
  const unsigned burst = plan_field(PH, offsetof(PlanHeader, burst));
  const uint32_t* upart = reinterpret_cast<const uint32_t*>(plan + plan_field(PH, offsetof(PlanHeader, groups_off)) +
                                                          burst * sizeof(DecodeToken));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) DecodeQ8Lds L;
  double* wgpart = reinterpret_cast<double*>(S.wgpart);
  const float* xg = reinterpret_cast<const float*>(plan + plan_field(PH, offsetof(PlanHeader, x_off)));
  const unsigned xs0 = 32 * ((unsigned)tid >> 2) + 8 * ((unsigned)tid & 3);
  const bool xin = ((unsigned)tid >> 2) < nsub;
  const unsigned sb0 = 2 * (unsigned)wave, sb1 = sb0 + 1;
  const bool has0 = sb0 < nsb, has1 = sb1 < nsb;
  const unsigned lb0 = min(sb0, nsb - 1), lb1 = min(sb1, nsb - 1);
  const uint32_t dq_off = 4608 * min(2 * (unsigned)wave + ((unsigned)lane >> 5), nsb - 1) + 32 * ((unsigned)lane & 31);
  const uint32_t dh_off =
      4608 * min(2 * (unsigned)wave + (((unsigned)lane & 15) >> 3), nsb - 1) + 4096 + 16 * ((unsigned)lane & 7);
  uint32_t bad = 0;

  unsigned p = blockIdx.x * tpw;
  const unsigned pend = min(p + tpw, np);
  PairBuf B = pair_buf(pairs + p);
  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  if (xin) {
    const float* xt = xg + (size_t)B.token * hidden + xs0;
    xv[0] = *reinterpret_cast<const float4*>(xt);
    xv[1] = *reinterpret_cast<const float4*>(xt + 4);
  }
  uint4 h0 = load_hdr(B, lb0, lane), h1 = load_hdr(B, lb1, lane);
  DecodeNib N[4];
  DecodeDnBytes D[4];
  load_nib(B, 0, lb0, lb1, lane, N[0]);
  load_dn(B, 0, dq_off, dh_off, D[0]);
  __builtin_amdgcn_sched_barrier(0);
  stage_x_q8(xv, 0, nsub, L, bad);
  __syncthreads();   // x is in LDS

  double y[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  const unsigned kg = (unsigned)lane >> 4, jcol = (unsigned)lane & 15;
  // As decode_kernel's unit loop, with every down after round 3 (h is
  // quantized over all 32 neurons); the next unit's first bytes are
  // requested during round 3 except its round-0 down bytes, requested after
  // this unit's downs have read D[0].
  for (unsigned k = 0;; ++k) {
    const unsigned q = p + 1, par = k & 1, t = par;
    const bool more = q < pend;
    const PairBuf Bn = pair_buf(pairs + (more ? q : p), more);
    load_nib(B, 1, lb0, lb1, lane, N[1]);
    load_dn(B, 1, dq_off, dh_off, D[1]);
    __builtin_amdgcn_sched_barrier(0);
    i32x4 b0[4], b1[4];
    double fx0[2], fx1[2];
    x_operands_q8(t, sb0, lane, L, b0, fx0);
    x_operands_q8(t, sb1, lane, L, b1, fx1);
    {
      double mp = 0.0;
      if (has0) mp += header_pass_q8(h0, sb0, 0, t, wave, lane, L, bad);
      if (has1) mp += header_pass_q8(h1, sb1, 1, t, wave, lane, L, bad);
      L.minp[par][wave][lane] = mp;
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const DecodeNib& Nc = N[rb];
      __builtin_amdgcn_sched_barrier(0);
      if (rb == 1 || rb == 2) {
        load_nib(B, rb + 1, lb0, lb1, lane, N[rb + 1]);
        load_dn(B, rb + 1, dq_off, dh_off, D[rb + 1]);
      } else if (rb == 3) {
        if (xin) {
          const float* xt = xg + (size_t)Bn.token * hidden + xs0;
          xv[0] = *reinterpret_cast<const float4*>(xt);
          xv[1] = *reinterpret_cast<const float4*>(xt + 4);
        }
        h0 = load_hdr(Bn, lb0, lane);
        h1 = load_hdr(Bn, lb1, lane);
        load_nib(Bn, 0, lb0, lb1, lane, N[0]);
      }
      __builtin_amdgcn_sched_barrier(0);
      double acc[4] = {0.0, 0.0, 0.0, 0.0};
      if (has0) rb_products_q8(Nc.q[0], b0, fx0, 0, rb, wave, lane, L, acc);
      if (has1) rb_products_q8(Nc.q[1], b1, fx1, 1, rb, wave, lane, L, acc);
      {
        const double r0 = row_sum_d(acc[0]), r1 = row_sum_d(acc[1]), r2 = row_sum_d(acc[2]), r3 = row_sum_d(acc[3]);
        if (jcol == 0) {
          double* rp = &L.rowp[par][wave][16 * rb + 4 * kg];
          *reinterpret_cast<double2*>(rp) = make_double2(r0, r1);
          *reinterpret_cast<double2*>(rp + 2) = make_double2(r2, r3);
        }
      }
      __syncthreads();   // every wavefront's sums of row-block rb are in LDS
      if (lane < 8) {
        const unsigned rg = 16 * rb + (unsigned)lane, ru = rg + 8;
        double a = 0.0, u = 0.0;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
          a += L.rowp[par][w][rg] - L.minp[par][w][rg];
          u += L.rowp[par][w][ru] - L.minp[par][w][ru];
        }
        // backends/ref.c:80-83: a and u narrowed to float, then SiLU in double.
        uint32_t hb = 0;
        const float af = narrow_dot(a), uf = narrow_dot(u);
        const float hv = silu_mul(af, uf, hb);
        if (wave == 0) bad |= hb;
        L.h[wave][8 * rb + lane] = hv;
      }
      __builtin_amdgcn_wave_barrier();
    }
    quantize_h32(L.h[wave], lane);   // backends/ref.c:85
#pragma unroll
    for (int r = 0; r < 4; ++r) down_round_q8(D[r], &L.h[wave][8 * r], wave, lane, nsb, L, y, bad);
    load_dn(Bn, 0, dq_off, dh_off, D[0]);
    store_partial_q8(wgpart, S.ustride, plan_read(upart + p), wave, lane, B.gate, y);
    if (!more) break;
    stage_x_q8(xv, par ^ 1, nsub, L, bad);
    __syncthreads();   // the next unit's x is in LDS
    p = q;
    B = Bn;
  }
  if (bad) flag(status, bad);
}

// Position p of a decode partial -> output column (see above).
__device__ __forceinline__ unsigned decode_column(unsigned p) {
  const unsigned w = p >> 9, hh = (p >> 8) & 1, l = (p >> 2) & 63, cc = p & 3;
  return 256 * (2 * w + (l >> 5)) + 8 * (l & 31) + 4 * hh + cc;
}

// Sum of a token's unit partials, 16 positions per workgroup (token =
// blockIdx.y, units [first, first + count) of the plan's token table), in
// fp64 and a fixed order: lane (q, ps) of wavefront w, ps = 16w + l/4, adds
// units ps, ps+64, ps+128, ps+192 of positions 16*blockIdx.x + 4q..4q+3 in
// that order (its four loads in flight together), a butterfly over the
// 16 ps of each wavefront combines them, and wavefront 0 adds the four
// wavefronts' sums in order. Narrowing follows the reference's overflow rule
// (backends/ref.c:95); the status word is decode_kernel's. A token's result
// depends only on its own units, in order.
constexpr int kReduceThreads = 256;
constexpr int kReducePositions = 16;
constexpr unsigned kReduceLanes = kReduceThreads / (kReducePositions / 4);   // 64 partial lanes
constexpr unsigned kReduceDepth = 4;                                          // units per partial lane
__device__ __forceinline__ double xor_d(double v, int m) {
  const int lo = __shfl_xor((int)(uint32_t)__double_as_longlong(v), m);
  const int hi = __shfl_xor((int)(uint32_t)((uint64_t)__double_as_longlong(v) >> 32), m);
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
// kDouble: the unit partials are doubles (decode_q8_kernel's).
template <bool kDouble>
__global__ __launch_bounds__(kReduceThreads) void decode_reduce(const uint8_t* __restrict__ plan, Scratch S) {
  (void)plan;
  const DecodeToken tk = S.A.tok[blockIdx.y];
  const unsigned hidden = S.A.hidden;
  uint32_t* status = S.ystat ? S.ystat : S.out + (size_t)S.parity * S.out_words;
  float* yout = (S.ystat || S.hstat ? S.yout : reinterpret_cast<float*>(status + 4)) + (size_t)blockIdx.y * hidden;
  if (S.ystat && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    const uint32_t e = *S.dstat;   // written by decode_kernel (kernel boundary)
    if (e) flag(status, e);
    *S.dstat = 0;                  // zero for the next static launch
  }
  const unsigned tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane & 3;
  const unsigned ps = 16 * wave + (lane >> 2);
  const unsigned p0 = kReducePositions * blockIdx.x + 4 * q;
  // Every load is issued unconditionally (units past the token's last read
  // its last unit again, and their values are then dropped), so that the
  // four are in flight together: a load under a lane condition is waited for
  // before the next one is issued.
  double v[4] = {0.0, 0.0, 0.0, 0.0};
  if constexpr (kDouble) {
    const double* part = reinterpret_cast<const double*>(S.wgpart);
    double2 r[kReduceDepth][2];
#pragma unroll
    for (unsigned k = 0; k < kReduceDepth; ++k) {
      const unsigned g = min(ps + kReduceLanes * k, tk.count - 1);
      const double2* src = reinterpret_cast<const double2*>(part + partial_index(tk.first + g, p0, S.ustride));
      r[k][0] = src[0];
      r[k][1] = src[1];
    }
#pragma unroll
    for (unsigned k = 0; k < kReduceDepth; ++k) {
      const bool in = ps + kReduceLanes * k < tk.count;
      v[0] += in ? r[k][0].x : 0.0;
      v[1] += in ? r[k][0].y : 0.0;
      v[2] += in ? r[k][1].x : 0.0;
      v[3] += in ? r[k][1].y : 0.0;
    }
  } else {
    float4 r[kReduceDepth];
#pragma unroll
    for (unsigned k = 0; k < kReduceDepth; ++k) {
      const unsigned g = min(ps + kReduceLanes * k, tk.count - 1);
      r[k] = *reinterpret_cast<const float4*>(S.wgpart + partial_index(tk.first + g, p0, S.ustride));
    }
#pragma unroll
    for (unsigned k = 0; k < kReduceDepth; ++k) {
      const bool in = ps + kReduceLanes * k < tk.count;
      v[0] += in ? (double)r[k].x : 0.0;
      v[1] += in ? (double)r[k].y : 0.0;
      v[2] += in ? (double)r[k].z : 0.0;
      v[3] += in ? (double)r[k].w : 0.0;
    }
  }
#pragma unroll
  for (int m = 4; m < 64; m <<= 1)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) v[cc] += xor_d(v[cc], m);
  __shared__ double red[kReduceThreads / 64][kReducePositions];
  if (lane < 4)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) red[wave][4 * q + cc] = v[cc];
  __syncthreads();
  if (tid < 64) {
    bool over = false;
    if (tid < kReducePositions) {
      const double t = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
      const unsigned col = decode_column(kReducePositions * blockIdx.x + tid);
      if (col < hidden) {
        float f = 0.f;
        if (!isfinite(t) || fabs(t) > (double)FLT_MAX) over = true;
        else f = (float)t;
        yout[col] = f;
      }
    }
    if (S.hstat) {
      // This workgroup's status word, written whether or not it is zero (the
      // host ORs them); workgroup (0, 0) adds decode_kernel's error bits and
      // zeroes them for the next launch.
      const bool any = __ballot(over) != 0;
      if (tid == 0) {
        uint32_t bits = any ? kErrRange : 0u;
        if (blockIdx.x == 0 && blockIdx.y == 0) {
          bits |= *S.dstat;   // written by decode_kernel (kernel boundary)
          *S.dstat = 0;
        }
        S.hstat[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = bits;
      }
    } else if (over) {
      flag(status, kErrRange);
    }
  }
}
static_assert(kDecodeUnitsPerToken <= kReduceDepth * kReduceLanes, "units per token within the reduce's lanes");
static_assert(kReduceThreads == 256, "the final sum adds four wavefronts");

// ------------------------------------------------- decode kernel, row formats
//
// F32 mode, every unit one of the row-format pairs (gate/up, down):
// (Q4_K, MXFP4) - the reference's native unit format -, (Q8_0, Q8_0) - also
// the shared expert -, (MXFP4, MXFP4) and (Q4_0, Q4_0). Same work list,
// unit partials and decode_reduce as decode_kernel: one workgroup of 8
// wavefronts per (token, pair) unit at a time, no h crossing workgroups.
//
// Gate/up: wavefront w takes neurons 4w..4w+3 (4 gate rows, then 4 up
// rows); lane c holds the row's columns 64c..64c+63 (the re-tiled lane
// chunks) and x of the same columns in registers, and the row's value is a
// wave-wide sum of the lanes' fp32 dots (lane_dot_f32, scales as the
// reference forms them, src/native.c:13-31). h = SiLU(a)*u in double
// (backends/ref.c:82-83) meets the other wavefronts in LDS.
//
// Down: thread (w, l) owns the 8 consecutive outputs 256*(2w + l/32) +
// 8*(l%32) + 0..7, exactly the 8 positions store_partial gives it, so the
// partial has decode_kernel's layout. Each output's 16- or 32-byte record
// over the 32 neurons (byte i: neuron i low nibble, 16+i high; Q8_0: two
// parts of 16 int8) is dotted with h in fp32, times its scale and the
// token's gate. The down bytes are requested halfway through the gate/up
// dots.
constexpr int kRowsWaveNeurons = kNeurons / kDecodeWaves;   // 4

struct RowsLds {
  float4 xq[16][kSubBlocks / 2];        // x of the unit's token in fp32, lane-major: [value/4 % 16][lane]
  int xl[4][2][2][kSubBlocks / 2][4];   // x of the unit's token as int8 digits, lane-major (stage_x)
  float xf[1][kSubBlocks];              // 2^e of each 32-value sub-block
  float xs[1][kSubBlocks];           // fp32 sum of each sub-block
  float xw[kSubBlocks][2];              // ref-q8: the two digits' weights s, u of each sub-block
  double xsd[kSubBlocks];               // ref-q8: exact sum of each sub-block's quantized values
  float h[kNeurons];
  float hmd;                            // q8_256: the d of the unit's quantized h
};

// The lane's x digits of sub-block 2c + J (J = 0, 1 of the lane's 64
// columns): digit d, dword i = values 4i..4i+3 of the sub-block.
struct LaneDigits {
  int q[4][8];
  float f;   // 2^e of the sub-block
  float s;   // fp32 sum of the sub-block
};

template <int J>
__device__ __forceinline__ void load_digits(const RowsLds& L, int c, LaneDigits& X) {
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int4 v = *reinterpret_cast<const int4*>(&L.xl[d][J][k][c][0]);
      X.q[d][4 * k] = v.x;
      X.q[d][4 * k + 1] = v.y;
      X.q[d][4 * k + 2] = v.z;
      X.q[d][4 * k + 3] = v.w;
    }
  X.f = L.xf[0][2 * c + J];
  X.s = L.xs[0][2 * c + J];
}

// sum_k w_k x_k over the sub-block from its four exact integer digit dots:
// x = 2^e (2^24 d0 + 2^16 d1 + 2^8 d2 + d3); each dot is below 2^24, so
// its conversion and the power-of-two weights are exact.
__device__ __forceinline__ float digit_sum(const int (&a)[4], float f) {
  return f * ((16777216.f * (float)a[0] + 65536.f * (float)a[1]) + (256.f * (float)a[2] + (float)a[3]));
}

// The lane's fp32 part of a row dot over sub-block 2c + J from exact
// integer dots (v_dot4_i32_i8 of the weights' integers and x's digits),
// scaled as the reference scales each weight (src/native.c:13-31): Q8_0
// d*q; Q4_K (d*sc)*q - dmin*m, the min term against the sub-block's fp32
// sum of x; Q4_0 d*(q-8), the offset against the same sum.
template <int type, int J>
__device__ __forceinline__ float lane_dot_digits(const LaneRaw& r, const float* sc, const float* mn,
                                                 const LaneDigits& X) {
  int acc[4] = {0, 0, 0, 0};
  if (type == TQ8_0) {
    // Part p: values 16p..16p+15 of the lane's 64; parts 2J, 2J+1 are the sub-block's.
#pragma unroll
    for (int p = 2 * J; p < 2 * J + 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int w = (int)word(r.q[p], i);
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[d] = __builtin_amdgcn_sdot4(w, X.q[d][4 * (p & 1) + i], acc[d], false);
      }
    return sc[J] * digit_sum(acc, X.f);
  }
  if (type == TQ4_K) {
    // Byte i of the 32-byte chunk: value i (low nibble, sub-block 2c) and
    // value 32+i (high nibble, sub-block 2c+1).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = word(r.q[i >> 2], i & 3);
      const int n = (int)(J ? nib_hi(v) : nib_lo(v));
#pragma unroll
      for (int d = 0; d < 4; ++d) acc[d] = __builtin_amdgcn_sdot4(n, X.q[d][i], acc[d], false);
    }
    return sc[J] * digit_sum(acc, X.f) - mn[J] * X.s;
  }
  // Q4_0: block J of the lane, byte i: value i (low nibble), 16+i (high).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = word(r.q[J], i);
    const int lo = (int)nib_lo(v), hi = (int)nib_hi(v);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc[d] = __builtin_amdgcn_sdot4(lo, X.q[d][i], acc[d], false);
      acc[d] = __builtin_amdgcn_sdot4(hi, X.q[d][4 + i], acc[d], false);
    }
  }
  return sc[J] * (digit_sum(acc, X.f) - 8.f * X.s);
}

struct RowsDown {
  uint4 q0[8], q1[8];   // records of the thread's 8 outputs (q1: Q8_0 second part)
  uint4 sc;             // their scales: 8 E8M0 bytes (MXFP4) or 8 fp16 (Q8_0, Q4_0)
};

template <int DN>
__device__ __forceinline__ void rows_load_down(const uint8_t* down, unsigned hidden, unsigned c0, RowsDown& R) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    R.q0[i] = ld16(down + 16 * (size_t)(c0 + i));
    if (DN == TQ8_0) R.q1[i] = ld16(down + 16 * (size_t)hidden + 16 * (size_t)(c0 + i));
  }
  if (DN == TMXFP4) {
    const uint64_t e = gld<uint64_t>(down + 16 * (size_t)hidden + c0);
    R.sc = make_uint4((uint32_t)e, (uint32_t)(e >> 32), 0u, 0u);
  } else {
    R.sc = ld16(down + (DN == TQ8_0 ? 32 : 16) * (size_t)hidden + 2 * (size_t)c0);
  }
}

// y[i] = gate * scale_i * sum_n W[c0+i][n] * h[n] for the thread's 8 outputs.
template <int DN>
__device__ __forceinline__ void rows_down(const RowsDown& R, const float* hs, float gate, bool valid, float (&y)[8],
                                          uint32_t& bad) {
  const float4* h4 = reinterpret_cast<const float4*>(hs);
  float hsum = 0.f;
  if (DN == TQ4_0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) hsum += (h4[i].x + h4[i].y) + (h4[i].z + h4[i].w);
  }
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    float sc;
    if (DN == TMXFP4) {
      const uint32_t e = (word(R.sc, o >> 2) >> (8 * (o & 3))) & 0xffu;
      if (valid && mx_blocks_bad(e, R.q0[o], 0u, R.q0[o])) bad |= kErrScale;
      sc = e8m0(e);
    } else {
      const uint32_t hb = (word(R.sc, o >> 1) >> (16 * (o & 1))) & 0xffffu;
      if (valid && half_bad(hb)) bad |= kErrScale;
      sc = half_to_float(hb);
    }
    float sum = 0.f;
    if (DN == TQ8_0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t v = word(i < 4 ? R.q0[o] : R.q1[o], i & 3);
        const float4 h = h4[i];
        sum = fmaf((float)(int8_t)v, h.x, sum);
        sum = fmaf((float)(int8_t)(v >> 8), h.y, sum);
        sum = fmaf((float)(int8_t)(v >> 16), h.z, sum);
        sum = fmaf((float)(int8_t)(v >> 24), h.w, sum);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = word(R.q0[o], i);
        const float4 a = h4[i], b = h4[4 + i];
        if (DN == TMXFP4) {
          const float2 e0 = fp4_pair(v, 1.0f, 0), e1 = fp4_pair(v, 1.0f, 1), e2 = fp4_pair(v, 1.0f, 2),
                       e3 = fp4_pair(v, 1.0f, 3);
          sum = fmaf(e0.x, a.x, sum);
          sum = fmaf(e1.x, a.y, sum);
          sum = fmaf(e2.x, a.z, sum);
          sum = fmaf(e3.x, a.w, sum);
          sum = fmaf(e0.y, b.x, sum);
          sum = fmaf(e1.y, b.y, sum);
          sum = fmaf(e2.y, b.z, sum);
          sum = fmaf(e3.y, b.w, sum);
        } else {
          const uint32_t lo = nib_lo(v), hi = nib_hi(v);
          sum = fmaf(ub(lo, 0), a.x, sum);
          sum = fmaf(ub(lo, 1), a.y, sum);
          sum = fmaf(ub(lo, 2), a.z, sum);
          sum = fmaf(ub(lo, 3), a.w, sum);
          sum = fmaf(ub(hi, 0), b.x, sum);
          sum = fmaf(ub(hi, 1), b.y, sum);
          sum = fmaf(ub(hi, 2), b.z, sum);
          sum = fmaf(ub(hi, 3), b.w, sum);
        }
      }
      if (DN == TQ4_0) sum -= 8.f * hsum;
    }
    // The reference forms gate * (W h) in fp64 (backends/ref.c:86-92): a zero
    // gate adds exactly nothing, and a product that only overflows fp32 in
    // the order sc * sum is formed as (gate * sc) * sum instead.
    const float t = sc * sum;
    y[o] = !valid || gate == 0.f ? 0.f : isfinite(t) ? gate * t : (gate * sc) * sum;
  }
}

// One unit: pair fields (uniform), x of the unit's token, gate/up rows, h
// through LDS, the down into y. MXFP4 rows dot in fp32 against x staged in
// LDS and held in registers (two codes per conversion); the integer formats
// dot in integers against x's digits staged in LDS.
template <int GU, int DN>
__device__ __forceinline__ uint32_t rows_unit(float* wgpart, unsigned ustride, unsigned unit, const PairDesc* P,
                                              const float* xg,
                                              unsigned hidden, int wave, int lane, RowsLds& L) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(P);
  const uint64_t slice = ((uint64_t)uniform(plan_read(w + 1)) << 32) | uniform(plan_read(w));
  const uint32_t proj = uniform(plan_read(w + 2));
  const uint32_t token = uniform(plan_read(w + 3)) >> 24;
  const float gate = __uint_as_float(uniform(plan_read(reinterpret_cast<const uint32_t*>(P->gate))));
  const int nch = (int)(hidden / 64);
  const unsigned nsub = hidden / 32;
  const bool active = lane < nch;
  const int c = active ? lane : 0;
  const unsigned n0 = kRowsWaveNeurons * (unsigned)wave;
  const unsigned cw = 256 * (2 * (unsigned)wave + ((unsigned)lane >> 5)) + 8 * ((unsigned)lane & 31);
  const bool dvalid = cw < hidden;
  const unsigned c0 = dvalid ? cw : 0;
  const uint8_t* down = reinterpret_cast<const uint8_t*>(slice) + 2 * (size_t)proj;
  constexpr bool kDigits = GU != TMXFP4;
  // The down bytes are requested halfway through the dots (after the gate
  // rows, or after the first sub-block pass, by when every row has
  // arrived): requested with the rows, they delay the rows the dots wait
  // for; requested after all dots, they arrive late (measured per call:
  // MXFP4 20.2 with the rows, 19.0 after, 17.9 halfway).
  const float* xt = xg + (size_t)token * hidden;
  uint32_t bad = 0;

  // x first, so that staging it waits for x alone: thread t holds values
  // 8t..8t+7, staged once per workgroup in LDS.
  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  float4 x[16];
  const unsigned tid = threadIdx.x;
  if ((tid >> 2) < nsub) {
    const float4* xs = reinterpret_cast<const float4*>(xt + 32 * (tid >> 2) + 8 * (tid & 3));
    xv[0] = xs[0];
    xv[1] = xs[1];
  }
  LaneRaw raw[2 * kRowsWaveNeurons];   // [gate rows][up rows]
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int i = 0; i < kRowsWaveNeurons; ++i) load_gu_row<GU>(slice, proj, k, n0 + i, nch, c, raw[kRowsWaveNeurons * k + i]);
  RowsDown R;
  if constexpr (!kDigits) {
    // Values 8t..8t+7 are float4s 2(t%8), 2(t%8)+1 of lane t/8's 64 values.
    if ((tid >> 2) < nsub) {
      L.xq[2 * (tid & 7)][tid >> 3] = xv[0];
      L.xq[2 * (tid & 7) + 1][tid >> 3] = xv[1];
    }
    __syncthreads();   // x is in LDS
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = L.xq[i][c];
  }
  float dot[2 * kRowsWaveNeurons];
  if constexpr (kDigits) {
    stage_x<RowsLds, true>(xv, 0, nsub, true, L, bad);
    __syncthreads();   // x's digits are in LDS
    // The lane's two sub-blocks in turn, every row each time: half the
    // digit registers of holding both.
    float part[2 * kRowsWaveNeurons];
    LaneDigits X;
    load_digits<0>(L, c, X);
#pragma unroll
    for (int r = 0; r < 2 * kRowsWaveNeurons; ++r) {
      float sc[2], mn[2];
      const bool ok = raw_scales<GU>(raw[r], c, sc, mn);
      if (active && !ok) bad |= kErrScale;
      part[r] = lane_dot_digits<GU, 0>(raw[r], sc, mn, X);
    }
    rows_load_down<DN>(down, hidden, c0, R);
    load_digits<1>(L, c, X);
#pragma unroll
    for (int r = 0; r < 2 * kRowsWaveNeurons; ++r) {
      float sc[2], mn[2];
      (void)raw_scales<GU>(raw[r], c, sc, mn);
      part[r] += lane_dot_digits<GU, 1>(raw[r], sc, mn, X);
      dot[r] = wave_total(active ? part[r] : 0.f);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 2 * kRowsWaveNeurons; ++r) {
      if (r == kRowsWaveNeurons) rows_load_down<DN>(down, hidden, c0, R);
      float sc[2], mn[2];
      const bool ok = raw_scales<GU>(raw[r], c, sc, mn);
      if (active && !ok) bad |= kErrScale;
      dot[r] = wave_total(active ? lane_dot_f32<GU>(raw[r], sc, mn, x, 0.f, 0.f) : 0.f);
    }
  }
  if (lane < kRowsWaveNeurons) {
    float a = dot[0], u = dot[kRowsWaveNeurons];
#pragma unroll
    for (int i = 1; i < kRowsWaveNeurons; ++i)
      if (lane == i) {
        a = dot[i];
        u = dot[kRowsWaveNeurons + i];
      }
    L.h[n0 + lane] = silu_mul(a, u, bad);
  }
  __syncthreads();   // the unit's 32 h are in LDS (and every lane has its digits)
  float y[8];
  rows_down<DN>(R, L.h, gate, dvalid, y, bad);
  store_partial(wgpart, ustride, unit, wave, lane, y);
  __syncthreads();   // h is read before the next unit writes it
  return bad;
}

// One instantiation per unit format: the routed pairs' (GA, DA) and the
// shared expert's (GB, DB); a launch runs both, each unit on its own.
template <int GA, int DA, int GB, int DB>
__global__ __launch_bounds__(kDecodeThreads) void decode_rows_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  const PlanHeader* PH = reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + plan_field(PH, offsetof(PlanHeader, pairs_off)));
  const unsigned hidden = plan_field(PH, offsetof(PlanHeader, hidden));
  const unsigned np = plan_field(PH, offsetof(PlanHeader, npairs)), tpw = plan_field(PH, offsetof(PlanHeader, tpw));
  const unsigned burst = plan_field(PH, offsetof(PlanHeader, burst));
  const uint32_t* upart = reinterpret_cast<const uint32_t*>(plan + plan_field(PH, offsetof(PlanHeader, groups_off)) +
                                                          burst * sizeof(DecodeToken));
  const float* xg = reinterpret_cast<const float*>(plan + plan_field(PH, offsetof(PlanHeader, x_off)));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) RowsLds L;
  uint32_t bad = 0;
  const unsigned pend = min((blockIdx.x + 1) * tpw, np);
  for (unsigned p = blockIdx.x * tpw; p < pend; ++p) {
    const PairDesc* P = pairs + p;
    // gu and dn are bytes 12 and 13 of the descriptor: word 3.
    const uint32_t w3 = uniform(plan_read(reinterpret_cast<const uint32_t*>(P) + 3));
    const uint32_t gu = w3 & 0xffu, dn = (w3 >> 8) & 0xffu;
    const unsigned unit = plan_read(upart + p);
    if (GA == GB && DA == DB) bad |= rows_unit<GA, DA>(S.wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
    else if (gu == GA && dn == DA) bad |= rows_unit<GA, DA>(S.wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
    else bad |= rows_unit<GB, DB>(S.wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
  }
  if (bad) flag(status, bad);
}

// ------------------------------------------------- row formats, ref-q8
//
// decode_rows_kernel's units in the ref-q8 arithmetic (see decode_q8_kernel)
// for the integer gate/up formats: the reference's native units (Q4_K
// gate/up, MXFP4 down, Q8_0 shared expert), all-Q8_0 and legacy Q4_0. x is
// staged as its two exact int8 digits (k, r), the v_dot4 dots per sub-block
// are exact integers, and everything after them is double: each lane's part
// of a row, the wave-wide sums, SiLU as ref forms it, h quantized over the
// unit's 32 neurons, the down (every MXFP4, Q8_0 and Q4_0 weight is exact in
// float) and the stored partial gate*dot.

struct LaneDigitsQ8 {
  int q[2][8];   // digits k, r of the sub-block, dword i = values 4i..4i+3
  float s, u;    // their weights
  double sum;    // exact sum of the sub-block's quantized values
};

template <int J, int kDigits = 2>
__device__ __forceinline__ void load_digits_q8(const RowsLds& L, int c, LaneDigitsQ8& X) {
#pragma unroll
  for (int d = 0; d < kDigits; ++d)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int4 v = *reinterpret_cast<const int4*>(&L.xl[d][J][k][c][0]);
      X.q[d][4 * k] = v.x;
      X.q[d][4 * k + 1] = v.y;
      X.q[d][4 * k + 2] = v.z;
      X.q[d][4 * k + 3] = v.w;
    }
  const float2 w = *reinterpret_cast<const float2*>(&L.xw[2 * c + J][0]);
  X.s = w.x;
  X.u = w.y;
  X.sum = L.xsd[2 * c + J];
}

// The lane's part of a row dot over sub-block 2c + J in double (scales as
// lane_dot_digits; sc and mn are exact floats).
template <int type, int J, int kDigits = 2>
__device__ __forceinline__ double lane_dot_digits_q8(const LaneRaw& r, const float* sc, const float* mn,
                                                     const LaneDigitsQ8& X) {
  int acc[2] = {0, 0};
  if (type == TQ8_0) {
#pragma unroll
    for (int p = 2 * J; p < 2 * J + 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int w = (int)word(r.q[p], i);
#pragma unroll
        for (int d = 0; d < kDigits; ++d) acc[d] = __builtin_amdgcn_sdot4(w, X.q[d][4 * (p & 1) + i], acc[d], false);
      }
  } else if (type == TQ4_K) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = word(r.q[i >> 2], i & 3);
      const int n = (int)(J ? nib_hi(v) : nib_lo(v));
#pragma unroll
      for (int d = 0; d < kDigits; ++d) acc[d] = __builtin_amdgcn_sdot4(n, X.q[d][i], acc[d], false);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = word(r.q[J], i);
      const int lo = (int)nib_lo(v), hi = (int)nib_hi(v);
#pragma unroll
      for (int d = 0; d < kDigits; ++d) {
        acc[d] = __builtin_amdgcn_sdot4(lo, X.q[d][i], acc[d], false);
        acc[d] = __builtin_amdgcn_sdot4(hi, X.q[d][4 + i], acc[d], false);
      }
    }
  }
  const double qx = (double)acc[0] * (double)X.s + (double)acc[1] * (double)X.u;   // sum of q * x, exact terms
  if (type == TQ4_K) return (double)sc[J] * qx - (double)mn[J] * X.sum;
  if (type == TQ4_0) return (double)sc[J] * (qx - 8.0 * X.sum);
  return (double)sc[J] * qx;
}

// dot[i] = hscale * sum_n W[c0+i][n] * h[n] in double for the thread's 8
// outputs (backends/ref.c:86-92 with h quantized, hscale 1; q8_256: h the
// codes, hscale their d); the gate is applied at the store.
template <int DN>
__device__ __forceinline__ void rows_down_q8(const RowsDown& R, const float* hs, double hscale, bool valid,
                                             double (&y)[8], uint32_t& bad) {
  const float4* h4 = reinterpret_cast<const float4*>(hs);
  double hsum = 0.0;
  if (DN == TQ4_0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) hsum += ((double)h4[i].x + (double)h4[i].y) + ((double)h4[i].z + (double)h4[i].w);
  }
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    float sc;
    if (DN == TMXFP4) {
      const uint32_t e = (word(R.sc, o >> 2) >> (8 * (o & 3))) & 0xffu;
      if (valid && mx_blocks_bad(e, R.q0[o], 0u, R.q0[o])) bad |= kErrScale;
      sc = e8m0(e);
    } else {
      const uint32_t hb = (word(R.sc, o >> 1) >> (16 * (o & 1))) & 0xffffu;
      if (valid && half_bad(hb)) bad |= kErrScale;
      sc = half_to_float(hb);
    }
    double sum = 0.0;
    if (DN == TQ8_0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t v = word(i < 4 ? R.q0[o] : R.q1[o], i & 3);
        const float4 h = h4[i];
        sum = fma((double)(int8_t)v, (double)h.x, sum);
        sum = fma((double)(int8_t)(v >> 8), (double)h.y, sum);
        sum = fma((double)(int8_t)(v >> 16), (double)h.z, sum);
        sum = fma((double)(int8_t)(v >> 24), (double)h.w, sum);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = word(R.q0[o], i);
        const float4 a = h4[i], b = h4[4 + i];
        if (DN == TMXFP4) {
          const float2 e0 = fp4_pair(v, 1.0f, 0), e1 = fp4_pair(v, 1.0f, 1), e2 = fp4_pair(v, 1.0f, 2),
                       e3 = fp4_pair(v, 1.0f, 3);
          sum = fma((double)e0.x, (double)a.x, sum);
          sum = fma((double)e1.x, (double)a.y, sum);
          sum = fma((double)e2.x, (double)a.z, sum);
          sum = fma((double)e3.x, (double)a.w, sum);
          sum = fma((double)e0.y, (double)b.x, sum);
          sum = fma((double)e1.y, (double)b.y, sum);
          sum = fma((double)e2.y, (double)b.z, sum);
          sum = fma((double)e3.y, (double)b.w, sum);
        } else {
          const uint32_t lo = nib_lo(v), hi = nib_hi(v);
          sum = fma((double)ub(lo, 0), (double)a.x, sum);
          sum = fma((double)ub(lo, 1), (double)a.y, sum);
          sum = fma((double)ub(lo, 2), (double)a.z, sum);
          sum = fma((double)ub(lo, 3), (double)a.w, sum);
          sum = fma((double)ub(hi, 0), (double)b.x, sum);
          sum = fma((double)ub(hi, 1), (double)b.y, sum);
          sum = fma((double)ub(hi, 2), (double)b.z, sum);
          sum = fma((double)ub(hi, 3), (double)b.w, sum);
        }
      }
      if (DN == TQ4_0) sum -= 8.0 * hsum;
    }
    y[o] = valid ? (double)sc * sum * hscale : 0.0;
  }
}

// kQ256: the AVX2 arithmetic (one int8 code per x value, group 256; SiLU in
// float; h codes and their d), otherwise ref-q8.
template <int GU, int DN, bool kQ256>
__device__ __forceinline__ uint32_t rows_unit_q8(double* wgpart, unsigned ustride, unsigned unit, const PairDesc* P,
                                                 const float* xg, unsigned hidden, int wave, int lane, RowsLds& L) {
  static_assert(GU != TMXFP4, "ref-q8 row units dot in integers");
  static_assert(!kQ256 || GU != TQ4_0, "q8_256 row units are native or Q8_0");
  constexpr int kDigits = kQ256 ? 1 : 2;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(P);
  const uint64_t slice = ((uint64_t)uniform(plan_read(w + 1)) << 32) | uniform(plan_read(w));
  const uint32_t proj = uniform(plan_read(w + 2));
  const uint32_t token = uniform(plan_read(w + 3)) >> 24;
  const float gate = __uint_as_float(uniform(plan_read(reinterpret_cast<const uint32_t*>(P->gate))));
  const int nch = (int)(hidden / 64);
  const unsigned nsub = hidden / 32;
  const bool active = lane < nch;
  const int c = active ? lane : 0;
  const unsigned n0 = kRowsWaveNeurons * (unsigned)wave;
  const unsigned cw = 256 * (2 * (unsigned)wave + ((unsigned)lane >> 5)) + 8 * ((unsigned)lane & 31);
  const bool dvalid = cw < hidden;
  const unsigned c0 = dvalid ? cw : 0;
  const uint8_t* down = reinterpret_cast<const uint8_t*>(slice) + 2 * (size_t)proj;
  const float* xt = xg + (size_t)token * hidden;
  uint32_t bad = 0;

  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  const unsigned tid = threadIdx.x;
  if ((tid >> 2) < nsub) {
    const float4* xs = reinterpret_cast<const float4*>(xt + 32 * (tid >> 2) + 8 * (tid & 3));
    xv[0] = xs[0];
    xv[1] = xs[1];
  }
  LaneRaw raw[2 * kRowsWaveNeurons];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int i = 0; i < kRowsWaveNeurons; ++i) load_gu_row<GU>(slice, proj, k, n0 + i, nch, c, raw[kRowsWaveNeurons * k + i]);
  RowsDown R;
  if constexpr (kQ256) stage_x_q256(xv, nsub, L, bad);
  else stage_x_q8<RowsLds, true>(xv, 0, nsub, L, bad);
  __syncthreads();   // x's digits are in LDS
  double part[2 * kRowsWaveNeurons];
  LaneDigitsQ8 X;
  load_digits_q8<0, kDigits>(L, c, X);
#pragma unroll
  for (int r = 0; r < 2 * kRowsWaveNeurons; ++r) {
    float sc[2], mn[2];
    const bool ok = raw_scales<GU>(raw[r], c, sc, mn);
    if (active && !ok) bad |= kErrScale;
    if (!kQ256 && GU == TQ4_K && active && !q4k_weights_exact(raw[r].h.x)) bad |= kErrInexact;
    part[r] = lane_dot_digits_q8<GU, 0, kDigits>(raw[r], sc, mn, X);
  }
  rows_load_down<DN>(down, hidden, c0, R);
  load_digits_q8<1, kDigits>(L, c, X);
  double dot[2 * kRowsWaveNeurons];
#pragma unroll
  for (int r = 0; r < 2 * kRowsWaveNeurons; ++r) {
    float sc[2], mn[2];
    (void)raw_scales<GU>(raw[r], c, sc, mn);
    part[r] += lane_dot_digits_q8<GU, 1, kDigits>(raw[r], sc, mn, X);
    dot[r] = wave_total(active ? part[r] : 0.0);
  }
  if (lane < kRowsWaveNeurons) {
    double a = dot[0], u = dot[kRowsWaveNeurons];
#pragma unroll
    for (int i = 1; i < kRowsWaveNeurons; ++i)
      if (lane == i) {
        a = dot[i];
        u = dot[kRowsWaveNeurons + i];
      }
    if constexpr (kQ256) L.h[n0 + lane] = silu_mul_q256(narrow_dot(a), narrow_dot(u), bad);
    else L.h[n0 + lane] = silu_mul(narrow_dot(a), narrow_dot(u), bad);   // backends/ref.c:80-83
  }
  __syncthreads();   // the unit's 32 h are in LDS
  if (wave == 0) {
    if constexpr (kQ256) quantize_h32_q256(L.h, &L.hmd, lane);   // backends/avx2.c:434
    else quantize_h32(L.h, lane);                                // backends/ref.c:85
  }
  __syncthreads();   // quantized
  double y[8];
  rows_down_q8<DN>(R, L.h, kQ256 ? (double)L.hmd : 1.0, dvalid, y, bad);
  store_partial_q8(wgpart, ustride, unit, wave, lane, gate, y);
  __syncthreads();   // h is read before the next unit writes it
  return bad;
}

template <int GA, int DA, int GB, int DB, bool kQ256 = false>
__global__ __launch_bounds__(kDecodeThreads) void decode_rows_q8_kernel(const uint8_t* __restrict__ plan, Scratch S) {
  const PlanHeader* PH = reinterpret_cast<const PlanHeader*>(plan);
  uint32_t* status = decode_status(S);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(plan + plan_field(PH, offsetof(PlanHeader, pairs_off)));
  const unsigned hidden = plan_field(PH, offsetof(PlanHeader, hidden));
  const unsigned np = plan_field(PH, offsetof(PlanHeader, npairs)), tpw = plan_field(PH, offsetof(PlanHeader, tpw));
  const unsigned burst = plan_field(PH, offsetof(PlanHeader, burst));
  const uint32_t* upart = reinterpret_cast<const uint32_t*>(plan + plan_field(PH, offsetof(PlanHeader, groups_off)) +
                                                          burst * sizeof(DecodeToken));
  const float* xg = reinterpret_cast<const float*>(plan + plan_field(PH, offsetof(PlanHeader, x_off)));
  double* wgpart = reinterpret_cast<double*>(S.wgpart);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) RowsLds L;
  uint32_t bad = 0;
  const unsigned pend = min((blockIdx.x + 1) * tpw, np);
  for (unsigned p = blockIdx.x * tpw; p < pend; ++p) {
    const PairDesc* P = pairs + p;
    const uint32_t w3 = uniform(plan_read(reinterpret_cast<const uint32_t*>(P) + 3));
    const uint32_t gu = w3 & 0xffu, dn = (w3 >> 8) & 0xffu;
    const unsigned unit = plan_read(upart + p);
    if (GA == GB && DA == DB) bad |= rows_unit_q8<GA, DA, kQ256>(wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
    else if (gu == GA && dn == DA) bad |= rows_unit_q8<GA, DA, kQ256>(wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
    else bad |= rows_unit_q8<GB, DB, kQ256>(wgpart, S.ustride, unit, P, xg, hidden, wave, lane, L);
  }
  if (bad) flag(status, bad);
}

// ------------------------------------------------------- load re-tiling
//
// dst[o] = src[source(o)] for every byte o of a slice; the permutations are
// the layouts documented above. One workgroup per slice.

struct SliceShape {
  uint32_t hidden, gu, dn, proj, down, slice;
};

__device__ __forceinline__ uint32_t gu_source(uint8_t type, uint32_t nch, uint32_t o) {
  // o is a byte offset inside one re-tiled gate/up row of 64*nch columns.
  if (type == TQ4_K) {
    if (o < 32 * nch) {
      uint32_t p = o / (16 * nch), r = o % (16 * nch), c = r / 16, i = r % 16;
      uint32_t sb = c / 4, k = c % 4;
      return 144 * sb + 16 + 32 * k + 16 * p + i;
    }
    uint32_t r = o - 32 * nch;
    return 144 * (r / 16) + r % 16;
  }
  if (type == TQ8_0) {
    if (o < 64 * nch) {
      uint32_t p = o / (16 * nch), r = o % (16 * nch), c = r / 16, i = r % 16;
      return 34 * (2 * c + p / 2) + 2 + 16 * (p % 2) + i;
    }
    uint32_t r = o - 64 * nch, c = r / 4, k = r % 4;
    return 34 * (2 * c + k / 2) + k % 2;
  }
  if (type == TMXFP4) {
    if (o < 32 * nch) {
      uint32_t p = o / (16 * nch), r = o % (16 * nch), c = r / 16, i = r % 16;
      return 17 * (2 * c + p) + 1 + i;
    }
    uint32_t r = o - 32 * nch, c = r / 2, p = r % 2;
    return 17 * (2 * c + p);
  }
  // Q4_0
  if (o < 32 * nch) {
    uint32_t p = o / (16 * nch), r = o % (16 * nch), c = r / 16, i = r % 16;
    return 18 * (2 * c + p) + 2 + i;
  }
  uint32_t r = o - 32 * nch, c = r / 4, k = r % 4;
  return 18 * (2 * c + k / 2) + k % 2;
}

// Byte o of a re-tiled [H x 32] down matrix.
__device__ __forceinline__ uint32_t down_source(uint8_t dn, uint32_t hidden, uint32_t o) {
  if (dn == TMXFP4) return o < 16 * hidden ? 17 * (o / 16) + 1 + o % 16 : 17 * (o - 16 * hidden);
  if (dn == TQ8_0) {
    if (o < 32 * hidden) {
      uint32_t p = o / (16 * hidden), r = o % (16 * hidden);
      return 34 * (r / 16) + 2 + 16 * p + r % 16;
    }
    uint32_t r = o - 32 * hidden;
    return 34 * (r / 2) + r % 2;
  }
  // Q4_0
  if (o < 16 * hidden) return 18 * (o / 16) + 2 + o % 16;
  uint32_t r = o - 16 * hidden;
  return 18 * (r / 2) + r % 2;
}

// Nibble (neuron n, column j) of a native transposed Q4_K down whose first
// byte is src[base]. Src is a byte source: a pointer or the generator below.
template <class Src>
__device__ __forceinline__ uint32_t q4kt_nibble(const Src& src, uint32_t base, uint32_t row_bytes, uint32_t n,
                                                uint32_t j) {
  const uint32_t b = base + n * row_bytes + 144 * (j / 256);
  uint32_t jj = j % 256, chunk = jj / 64, i = jj % 32, half = (jj % 64) / 32;
  return (src[b + 16 + 32 * chunk + i] >> (4 * half)) & 15u;
}

template <class Src>
__device__ __forceinline__ uint8_t q4kt_byte(const Src& src, uint32_t base, uint32_t hidden, uint32_t o) {
  const uint32_t row_bytes = 144 * (hidden / 256);
  uint32_t sb = o / 4608, r = o % 4608;
  if (r >= 4096) {
    uint32_t n = (r - 4096) / 16, i = (r - 4096) % 16;
    return src[base + n * row_bytes + 144 * sb + i];
  }
  uint32_t k = r / 1024, l = (r % 1024) / 16, m = r % 16, wd = m / 4, bb = m % 4;
  uint32_t n = 8 * k + 2 * wd + bb / 2;
  uint32_t j = 256 * sb + 4 * l + 2 * (bb % 2);
  return (uint8_t)(q4kt_nibble(src, base, row_bytes, n, j) | (q4kt_nibble(src, base, row_bytes, n, j + 1) << 4));
}

// Byte o of the TQ4_KM gate/up tiles of a pair (layout above) from the
// reference rows: gate rows at 0, up rows at proj, row n at n * 144 * nsb,
// super-block sb at 144 * sb with its 128 nibble bytes from offset 16
// (element j of a super-block: byte 32 * (j / 64) + j % 32, high nibble when
// j % 64 >= 32).
template <class Src>
__device__ __forceinline__ uint8_t km_byte(const Src& src, uint32_t hidden, uint32_t proj, uint32_t o) {
  const uint32_t row_bytes = 144 * (hidden / 256), sb = o / 9216, r = o % 9216;
  if (r < 1024) {
    const uint32_t rb = r / 256, i = (r / 16) % 16;
    return src[(i >> 3) * proj + (8 * rb + (i & 7)) * row_bytes + 144 * sb + r % 16];
  }
  const uint32_t q = r - 1024, rb = q / 2048, p = (q / 1024) & 1, lane = (q / 16) & 63, byte = q & 15;
  const uint32_t i = lane & 15, kg = lane >> 4, u = byte >> 2, b = byte & 3;
  const uint32_t base = (i >> 3) * proj + (8 * rb + (i & 7)) * row_bytes + 144 * sb + 16;
  const uint32_t j0 = 32 * (4 * p + kg) + 8 * u + b, j1 = j0 + 4;   // positions of the low and high nibble
  const uint32_t n0 = (src[base + 32 * (j0 / 64) + j0 % 32] >> (4 * ((j0 % 64) / 32))) & 15u;
  const uint32_t n1 = (src[base + 32 * (j1 / 64) + j1 % 32] >> (4 * ((j1 % 64) / 32))) & 15u;
  return (uint8_t)(n0 | (n1 << 4));
}

// Byte o of a re-tiled slice whose reference-layout bytes are src[0..).
template <class Src>
__device__ uint8_t retile_byte(const SliceShape& s, const Src& src, uint32_t o) {
  const uint32_t nch = s.hidden / 64;
  if (o < 2 * s.proj && s.gu == TQ4_KM) return km_byte(src, s.hidden, s.proj, o);
  if (o < 2 * s.proj) {
    uint32_t row_bytes = s.proj / kNeurons, rbase = (o / row_bytes) * row_bytes;
    return src[rbase + gu_source((uint8_t)s.gu, nch, o - rbase)];
  }
  uint32_t od = o - 2 * s.proj;
  if (s.dn == TQ4_KT) return q4kt_byte(src, 2 * s.proj, s.hidden, od);
  return src[2 * s.proj + down_source((uint8_t)s.dn, s.hidden, od)];
}

// ------------------------------------------------------------ synthetic data
//
// Measurement weights generated on the device: every byte of a slice in the
// reference layout is a pure function of (seed, block, layer, expert, byte
// offset), so the generator is a byte source for retile_byte and writes the
// re-tiled block directly. Distributions: Q4_K nibbles and 6-bit scales
// uniform, d and dmin = fp16(U[1e-3, 1e-2]); Q8_0 int8 uniform on [-127, 127]
// with an fp16(U[1e-3, 1e-2]) scale; MXFP4 codes uniform, E8M0 uniform on
// [118, 130]; Q4_0 nibbles uniform with an fp16(U[1e-3, 1e-2]) scale. The hash
// is the splitmix64 finaliser (Steele, Lea, Flood 2014).
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t synth_hash(uint64_t key, unsigned domain, uint64_t word) {
  return mix64(key ^ ((uint64_t)domain << 60) ^ word);
}

// fp16 bits of 1e-3 + 9e-3*u (u = top 24 bits of h / 2^24), round to nearest
// even. Explicitly rounded fp64 operations: no contraction into an fma.
__device__ __forceinline__ uint16_t synth_scale(uint64_t h) {
  const double u = (double)(h >> 40) * 0x1p-24;
  const double v = __dadd_rn(1e-3, __dmul_rn(9e-3, u));
  const uint64_t bits = (uint64_t)__double_as_longlong(v);
  int e = (int)((bits >> 52) & 0x7ff) - 1023 + 15;
  uint64_t mant = bits & ((1ull << 52) - 1), q = mant >> 42, rem = mant & ((1ull << 42) - 1);
  if (rem > (1ull << 41) || (rem == (1ull << 41) && (q & 1))) ++q;
  if (q == 1024) {
    q = 0;
    ++e;
  }
  return (uint16_t)((unsigned)e << 10 | (unsigned)q);
}

__device__ __forceinline__ uint32_t type_block_bytes(uint32_t type) {
  return type == TQ4_K ? 144 : type == TQ8_0 ? 34 : type == TMXFP4 ? 17 : 18;
}

__device__ __forceinline__ uint8_t synth_block_byte(uint32_t type, uint64_t key, uint32_t s, uint32_t k) {
  const uint32_t o = s + k;
  if (type == TQ4_K) {
    if (k < 4) {
      const uint16_t h = synth_scale(synth_hash(key, 1, s + (k & 2)));
      return (uint8_t)(k & 1 ? h >> 8 : h);
    }
  } else if (type == TQ8_0) {
    if (k < 2) {
      const uint16_t h = synth_scale(synth_hash(key, 1, s));
      return (uint8_t)(k & 1 ? h >> 8 : h);
    }
    return (uint8_t)(int8_t)((int)((synth_hash(key, 2, o) >> 32) % 255u) - 127);
  } else if (type == TMXFP4) {
    if (k == 0) return (uint8_t)(118 + (synth_hash(key, 1, s) >> 32) % 13u);
  } else if (k < 2) {
    const uint16_t h = synth_scale(synth_hash(key, 1, s));
    return (uint8_t)(k & 1 ? h >> 8 : h);
  }
  return (uint8_t)(synth_hash(key, 0, o >> 3) >> (8 * (o & 7)));
}

// Byte source: slice bytes in the reference layout, generated on demand.
struct SynthSrc {
  uint64_t key;
  uint32_t gu, dn;            // block types of gate/up rows and of down rows
  uint32_t proj, gu_row, dn_row;
  __device__ __forceinline__ uint8_t operator[](uint32_t o) const {
    if (o < 2 * proj) {
      const uint32_t rl = (o < proj ? o : o - proj) % gu_row, k = rl % type_block_bytes(gu);
      return synth_block_byte(gu, key, o - k, k);
    }
    const uint32_t k = (o - 2 * proj) % dn_row % type_block_bytes(dn);
    return synth_block_byte(dn, key, o - k, k);
  }
};

__host__ __device__ __forceinline__ uint64_t synth_key(uint64_t seed, uint32_t block, uint32_t layer, uint32_t expert) {
  return mix64(seed) ^ ((uint64_t)block << 54) ^ ((uint64_t)layer << 44) ^ ((uint64_t)expert << 32);
}

// Slices [first, first+count) of consecutive layout: routed slices of one
// shape; `shared_every` marks the shared slice position (513th of a layer).
__global__ void retile_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, SliceShape routed,
                              SliceShape shared, uint64_t layer_bytes, uint32_t first_slice, uint32_t nslices) {
  uint32_t sidx = first_slice + blockIdx.x;
  if (blockIdx.x >= nslices) return;
  uint32_t layer = sidx / 513, e = sidx % 513;
  uint64_t off = layer * layer_bytes + (uint64_t)e * routed.slice;
  const SliceShape& s = e == kShared ? shared : routed;
  const uint8_t* in = src + off;
  uint8_t* out = dst + off;
  for (uint32_t o = threadIdx.x; o < s.slice; o += blockDim.x) out[o] = retile_byte(s, in, o);
}

// Synthetic slices [first, first+n) written re-tiled into dst (one workgroup
// per slice, four bytes per thread and step; slice sizes are multiples of 16).
__global__ void synth_kernel(uint8_t* __restrict__ dst, SliceShape routed, SliceShape shared, uint64_t layer_bytes,
                             uint32_t first_slice, uint32_t nslices, uint64_t seed, uint32_t block) {
  if (blockIdx.x >= nslices) return;
  const uint32_t sidx = first_slice + blockIdx.x, layer = sidx / 513, e = sidx % 513;
  const bool sh = e == kShared;
  const SliceShape& s = sh ? shared : routed;
  SynthSrc src;
  src.key = synth_key(seed, block, layer, e);
  src.gu = s.gu == TQ4_KM ? TQ4_K : s.gu;
  src.dn = s.dn == TQ4_KT ? TQ4_K : s.dn;
  src.proj = s.proj;
  src.gu_row = s.proj / kNeurons;
  src.dn_row = s.dn == TQ4_KT ? (s.hidden / 256) * 144 : type_block_bytes(s.dn);
  uint32_t* out = reinterpret_cast<uint32_t*>(dst + layer * layer_bytes + (uint64_t)e * routed.slice);
  for (uint32_t w = threadIdx.x; w < s.slice / 4; w += blockDim.x) {
    uint32_t v = 0;
    for (uint32_t i = 0; i < 4; ++i) v |= (uint32_t)retile_byte(s, src, 4 * w + i) << (8 * i);
    out[w] = v;
  }
}

// ------------------------------------------------------------ prefill path
// A prefill chunk: T tokens of one layer (T up to kMaxBatchTokens), each with
// its own top-10 routing, F32; every owned slice Q4_K with the transposed
// down, or every one a native unit (row-format kernels further below), and
// the shared expert on the tokens whose gate asks for it. The reference
// serves it as run() calls of at most 8 tokens (client/fronk_client.h:41-42,
// src/backend.h:21); the result of token t is that of run() on token t alone
// (backends/ref.c:57-98). Here the tokens are grouped by routed expert, so
// that each expert's weights are read once for all of its tokens and the
// work is a contraction:
//   prefill_split    (token): x as two f16 parts of x * 2^-e, once;
//   prefill_gate_up  (tile, slice): a, u of up to 16 tokens over one slice's
//                    32 neurons on f16 matrix cores (operands exact), then
//                    gate*SiLU(a)*u;
//   prefill_down     (tile, 512 outputs): the expert's down matrix over all
//                    owned slices applied to the tile's h on f16 matrix
//                    cores (A = sc*q exact, B = d*h in two exact parts), one
//                    fp32 partial per (token, expert);
//   prefill_reduce   (token, 1024 outputs): the token's 10 expert partials
//                    (then the shared expert's) summed in its routing order
//                    in fp64, then narrowed with the reference's rule
//                    (backends/ref.c:37-40, 95).
// Matrix-core layouts used below (16x16 tiles, 64 lanes): v_mfma_f32_16x16x32
// (f16/bf16): A lane l holds row l%16, k = 8(l/16)..+7; B lane l holds
// column l%16, the same k; C lane l holds rows 4(l/16)..+3 of column l%16.
// v_mfma_f32_16x16x4_f32 (the min terms): A lane l holds A[l%16][l/16], B
// lane l B[l/16][l%16].
constexpr int kTileTokens = 16;          // tokens of one expert tile (the MFMA N)
constexpr int kBatchThreads = 512;
constexpr int kMaxBatchTokens = 4096;
constexpr int kDownCols = 1024;          // outputs of one prefill_down workgroup

struct BatchTile {                       // one routed expert and up to 16 of its tokens
  uint32_t expert, ntok, slot0, pad;
};
struct BatchSlot {                       // one (token, expert) of the chunk
  uint32_t token;
  float gate;
};
struct BatchHeader {
  uint32_t hidden, tokens, nslots, ntiles;   // ntiles: routed tiles (the shared expert's follow)
  uint32_t nblk, layer, tiles_off, slots_off;
  uint32_t tokslot_off, x_off, total, experts;
  uint32_t nshared, shtiles, gu, dn;         // tokens with the shared expert, its tiles; routed formats
  uint64_t slice_bytes, proj, shared_proj;
  uint64_t base[kBlocks];                // owned slices in ascending block order: the layer's base
};
static_assert(sizeof(BatchHeader) == 248, "batch header layout");
constexpr uint32_t kNoSlot = ~0u;        // tokslot entry of a token without the shared expert
struct BatchScratch {
  float* h;                              // [nslots][nblk * 32] gate * h
  float* part;                           // [nslots][hidden] per-(token, expert) partials
  float* y;                              // [tokens][hidden]
  uint16_t* xh;                          // [tokens][super-block][2 parts][256] x' = x * 2^-e as f16 hi, lo
  float* dscale;                         // [tokens] 2^e
  float* dsum;                           // [tokens][super-block][8] sub-block sums of x'
  uint32_t* status;
};

// x of the chunk for the f16 matrix cores: per token, x' = x * 2^-e with 2^e
// chosen so that |x'| < 2^15, written as two f16 parts hi = f16(x'),
// lo = f16(x' - hi) (22 significant bits; the f16 subnormal floor 2^-24 is
// 2^-39 of the token's largest value), plus 2^e and the fp32 sum of each
// 32-value sub-block of x' (for the min terms).
__global__ __launch_bounds__(1024) void prefill_split(const uint8_t* __restrict__ plan, BatchScratch S) {
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  const unsigned t = blockIdx.x, hidden = H.hidden, nsb = hidden / 256, v0 = 4 * threadIdx.x;
  const bool live = v0 < hidden;
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) x = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(plan + H.x_off) + (size_t)t * hidden + v0);
  __shared__ float red[16];
  __shared__ uint32_t nonfinite;
  if (threadIdx.x == 0) nonfinite = 0;
  float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  const bool fin = isfinite(x.x) && isfinite(x.y) && isfinite(x.z) && isfinite(x.w);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  __syncthreads();
  if (!fin) nonfinite = 1;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = 0.f;
#pragma unroll
  for (int w = 0; w < 16; ++w) m = fmaxf(m, red[w]);
  const bool ok = nonfinite == 0;
  int E = 0;
  if (ok && m > 0.f) (void)frexpf(m, &E);   // m < 2^E
  const int e = max(E - 15, -126);
  const float v[4] = {x.x, x.y, x.z, x.w};
  float xs[4];
  _Float16 hi[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xs[j] = ok ? ldexpf(v[j], -e) : 0.f;
    hi[j] = (_Float16)xs[j];
    lo[j] = (_Float16)(xs[j] - (float)hi[j]);
  }
  float s = (xs[0] + xs[1]) + (xs[2] + xs[3]);
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);   // the 8 threads of a 32-value sub-block
  if (live) {
    const unsigned sb = v0 / 256, pos = v0 % 256;
    uint16_t* dst = S.xh + ((size_t)t * nsb + sb) * 512 + pos;
    *reinterpret_cast<uint2*>(dst) = make_uint2(
        (uint32_t)__builtin_bit_cast(uint16_t, hi[0]) | (uint32_t)__builtin_bit_cast(uint16_t, hi[1]) << 16,
        (uint32_t)__builtin_bit_cast(uint16_t, hi[2]) | (uint32_t)__builtin_bit_cast(uint16_t, hi[3]) << 16);
    *reinterpret_cast<uint2*>(dst + 256) = make_uint2(
        (uint32_t)__builtin_bit_cast(uint16_t, lo[0]) | (uint32_t)__builtin_bit_cast(uint16_t, lo[1]) << 16,
        (uint32_t)__builtin_bit_cast(uint16_t, lo[2]) | (uint32_t)__builtin_bit_cast(uint16_t, lo[3]) << 16);
    if ((threadIdx.x & 7) == 0) S.dsum[((size_t)t * nsb + sb) * 8 + pos / 32] = s;
  }
  if (threadIdx.x == 0) {
    S.dscale[t] = ldexpf(1.f, e);
    if (!ok) flag(S.status, kErrRange);   // a non-finite x makes the token's a and u non-finite
  }
}

// LDS bytes per (part, token) row: 512 + 16 of padding, so that the rows of
// 8 consecutive tokens start 16 bytes apart modulo 128 and a 16-byte read
// across them touches every bank once.
constexpr int kXhRow = 528;

struct GateUpLds {
  uint8_t xh[2][2][kTileTokens][kXhRow];     // [buffer][part][token][256 f16]: one super-block of x'
  float xs[2][kTileTokens][8];               // sub-block sums of x'
  float main[kDecodeWaves][16][kTileTokens]; // [wave][row][token] scale-weighted dot part
  float mins[kDecodeWaves][16][kTileTokens]; // [wave][row][token] min part
};


// Workgroup (tile, slice): wavefront w takes row-block w%4 (gate rows of
// neurons 8rb..8rb+7, then their up rows) and part w/4 (sub-blocks 0-3 or 4-7
// of every super-block) of the TQ4_KM tiles; lane 16kg + i holds sub-block
// 4p + kg of row i, which makes it the B operand of v_mfma_f32_16x16x32_f16
// (column i, k = 8kg..8kg+7) for 8 positions at a time: B = sc*q, exact in
// f16, so that each MFMA sums over 4 sub-blocks at once and the super-block
// is scaled by d only once. A = x' in two f16 parts (two MFMAs), tokens as
// rows, so that the four results of a lane are one weight row's, scaled by
// that row's d from the lane's own header. The min terms,
// sum_sub dmin * m_sub * sum(x'_sub), take one fp32 MFMA per super-block; the
// token's 2^e multiplies a and u at the end. x' moves through LDS one
// super-block at a time, double-buffered.
__global__ __launch_bounds__(kBatchThreads, 4) void prefill_gate_up(const uint8_t* __restrict__ plan,
                                                                    BatchScratch S) {
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  // Workgroups go round-robin over the 8 XCDs; each XCD takes a contiguous
  // run of the (tile, slice) list, so that a tile's 20 slices read its x'
  // from one L2.
  const unsigned nblk = H.nblk, per = gridDim.x / 8, b = blockIdx.x;
  const unsigned j = b < 8 * per ? (b % 8) * per + b / 8 : b, brank = j % nblk;
  const BatchTile T = reinterpret_cast<const BatchTile*>(plan + H.tiles_off)[j / nblk];
  const BatchSlot* slots = reinterpret_cast<const BatchSlot*>(plan + H.slots_off) + T.slot0;
  const unsigned hidden = H.hidden, nsb = hidden / 256;
  const uint8_t* slice = reinterpret_cast<const uint8_t*>(H.base[brank] + (uint64_t)T.expert * H.slice_bytes);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const unsigned rb = (unsigned)wave & 3, p = (unsigned)wave >> 2, kg = (unsigned)lane >> 4,
                 col = (unsigned)lane & 15;
  __shared__ __align__(16) GateUpLds L;
  // Staging: thread -> token tl, 32-byte piece c of its 1 KB of x' (part
  // c/16, positions 16(c%16)..+15).
  const unsigned tl = (unsigned)tid >> 5, c = (unsigned)tid & 31;
  const bool live = tl < T.ntok;
  const size_t trow = (size_t)(live ? slots[tl].token : 0) * nsb;
  const uint16_t* xsrc = S.xh + trow * 512 + 16 * c;
  // x' runs two super-blocks ahead in two register sets, the weights three
  // ahead in three (the loop is unrolled by six so that no set is copied
  // while its loads are in flight; the last weight loads re-read super-block
  // nsb-1 rather than branch).
  struct XStage {
    uint4 d[2];
    float s;
  };
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  auto load_x = [&](unsigned s, XStage& X) {
    if (live) {
      X.d[0] = *reinterpret_cast<const uint4*>(xsrc + 512 * (size_t)s);
      X.d[1] = *reinterpret_cast<const uint4*>(xsrc + 512 * (size_t)s + 8);
      if (c < 8) X.s = S.dsum[(trow + s) * 8 + c];
    }
  };
  auto store_x = [&](unsigned buf, const XStage& X) {
    uint8_t* row = &L.xh[buf][c / 16][tl][32 * (c % 16)];
    *reinterpret_cast<uint4*>(row) = X.d[0];
    *reinterpret_cast<uint4*>(row + 16) = X.d[1];
    if (c < 8) L.xs[buf][tl][c] = X.s;
  };
  const uint8_t* wq = slice + 1024 + 2048 * rb + 1024 * p + 16 * (unsigned)lane;   // + 9216 s
  const uint8_t* wh = slice + 256 * rb + 16 * col;
  uint32_t bad = 0, hflag = 0;   // hflag: half_bad_bits of the scale words read
  struct WStage {
    uint4 q, h;
  };
  auto load_w = [&](unsigned s) {
    const size_t o = 9216 * (size_t)min(s, nsb - 1);
    return WStage{ld16(wq + o), ld16(wh + o)};
  };
  XStage xa = {{z4, z4}, 0.f}, xb = {{z4, z4}, 0.f};
  load_x(0, xa);
  WStage wa = load_w(0), wb = load_w(1), wc = load_w(2);
  store_x(0, xa);
  if (1 < nsb) load_x(1, xa);
  __syncthreads();
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  f32x4 cmin = {0.f, 0.f, 0.f, 0.f};
  // Super-block s: W holds its weights (reloaded with those of s+3 once
  // read), cur holds x' of s+1 (stored at the end), s+2 is loaded into nxt.
  auto step = [&](unsigned s, WStage& W, XStage& cur, XStage& nxt) {
    const unsigned buf = s & 1;
    const uint4 qc = W.q, hc = W.h;
    if (s + 2 < nsb) load_x(s + 2, nxt);
    uint32_t sc, mi;
    q4k_scale_min(hc.y, hc.z, hc.w, 4 * p + kg, sc, mi);
    const f16x2 sch = f16_pair(sc);
    hflag |= half_bad_bits(hc.x);
    const float d = half_to_float(hc.x & 0xffff);   // of row col, the lane's rows of the product
    // x' of token col, part h, sub-block 4p + kg at LDS
    // xh[buf][h][col][2 (32 (4p + kg) + 8v)].
    const uint8_t* xb8 = &L.xh[buf][0][col][64 * (4 * p + kg)];
    // The parts accumulate in tiles of their own: a lo product added to the
    // hi sum in the matrix core loses low bits that a neuron's dot, whose
    // main and min terms can nearly cancel, needs.
    f32x4 c_hi = {0.f, 0.f, 0.f, 0.f}, c_lo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      // Word v: low nibbles = positions 8v..8v+3, high nibbles 8v+4..8v+7.
      const uint32_t w = word(qc, v), lo = nib_lo(w), hi = nib_hi(w);
      const u32x4 aw = {nib_pair_sc<false>(lo, sch), nib_pair_sc<true>(lo, sch), nib_pair_sc<false>(hi, sch),
                        nib_pair_sc<true>(hi, sch)};
      const f16x8 a = __builtin_bit_cast(f16x8, aw);
      const uint4 bh = *reinterpret_cast<const uint4*>(xb8 + 16 * v);
      const uint4 bl = *reinterpret_cast<const uint4*>(xb8 + kTileTokens * kXhRow + 16 * v);
      c_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bh), a, c_hi, 0, 0, 0);
      c_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bl), a, c_lo, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, c_hi[r] + c_lo[r], acc[r]);
    // Min terms: A = the sub-block sum of token col, B = -dmin * m of the
    // lane's (sub-block, row).
    cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(L.xs[buf][col][4 * p + kg], -half_to_float(hc.x >> 16) * (float)mi,
                                                cmin, 0, 0, 0);
    W = load_w(s + 3);
    if (s + 1 < nsb) store_x(buf ^ 1, cur);
    __syncthreads();
  };
  for (unsigned s = 0; s < nsb; s += 6) {
    step(s, wa, xa, xb);
    if (s + 1 < nsb) step(s + 1, wb, xb, xa);
    if (s + 2 < nsb) step(s + 2, wc, xa, xb);
    if (s + 3 < nsb) step(s + 3, wa, xb, xa);
    if (s + 4 < nsb) step(s + 4, wb, xa, xb);
    if (s + 5 < nsb) step(s + 5, wc, xb, xa);
  }
  // The products are [token][row] (x' is the A operand, so that a lane's
  // four results share its row's d): lane (kg, col) holds tokens
  // 4kg..4kg+3 of row col.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    L.main[wave][col][4 * kg + r] = acc[r];
    L.mins[wave][col][4 * kg + r] = cmin[r];
  }
  __syncthreads();
  // Thread -> (row-block, neuron i, token n): a = gate row i, u = up row 8+i,
  // each (dot part + min part) of part 0, then of part 1, times 2^e.
  {
    const unsigned trb = (unsigned)tid >> 7, i = ((unsigned)tid >> 4) & 7, n = (unsigned)tid & 15;
    if (n < T.ntok) {
      const float sx = S.dscale[slots[n].token];
      const float a = ((L.main[trb][i][n] + L.mins[trb][i][n]) + (L.main[trb + 4][i][n] + L.mins[trb + 4][i][n])) * sx;
      const float u = ((L.main[trb][8 + i][n] + L.mins[trb][8 + i][n]) +
                       (L.main[trb + 4][8 + i][n] + L.mins[trb + 4][8 + i][n])) * sx;
      uint32_t hb = 0;
      const float h = slots[n].gate * silu_mul_f32(a, u, hb);
      bad |= hb;
      S.h[(size_t)(T.slot0 + n) * (nblk * kNeurons) + kNeurons * brank + 8 * trb + i] = h;
    }
  }
  if (hflag & kHalfBadBits) bad |= kErrScale;
  if (bad) flag(S.status, bad);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// v as three bf16 values whose sum is v exactly (8 + 8 + 8 significant bits,
// each residual exact in fp32).
__device__ __forceinline__ void split_bf16(const float (&v)[8], bf16x8& b1, bf16x8& b2, bf16x8& b3) {
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    b1[j] = (__bf16)v[j];
    r[j] = v[j] - (float)b1[j];
    b2[j] = (__bf16)r[j];
    r[j] -= (float)b2[j];
    b3[j] = (__bf16)r[j];
  }
}

// Workgroup (tile, 512 outputs), four wavefronts: wavefront w takes the 128
// outputs 256 sb + 128 hb .. +127 (sb = 2 blockIdx.y + w/2, hb = w%2), eight
// 16-output tiles in one pass over all owned slices (B, the slice's header
// table and the min terms formed once per slice for all eight; three
// workgroups per CU, so that the eight accumulators fit without spills). With the Q4_K-T down's weight
// w = d sc q - dmin m (src/native.c:14-22; per neuron n a super-block over
// the outputs, sub-block g of 32 outputs), a slice adds
//   sum_n d_n sc_ng q_on h'_n  -  sum_n dmin_n m_ng h'_n
// to output o of sub-block g, with h' = h * 2^-e_t (per token t of the tile,
// e_t puts the largest |h'| in [2^12, 2^13)). The first sum runs on
// v_mfma_f32_16x16x32_f16 over the 32 neurons (lane group kq: neurons
// 8kq..8kq+7):
//   A[o][n] = sc_ng * q_on exactly in f16 (sc q < 1024), a packed 16-bit
//     multiply-add and an f16 subtraction per two neurons (scaled_u16);
//   B[n][t] = d_n h'_nt in two f16 parts (22 significant bits), formed once
//     per slice for the wavefront's eight tiles;
// and the products add straight into the tiles' accumulators over the
// slices. The second sum is fp32 FMAs per (sub-block, token). A 16-byte unit
// holds 4 outputs x 8 neurons; each lane of a quad loads one of the four
// units its quad's four tiles need, and the quad shares them by DPP. A slice
// in which a neuron's |d| is 4 or more (d h' could leave f16's range; no real
// unit has such a d) is deferred to the end and taken with B scaled down by
// a power of two.
constexpr float kDownDirect = 4.f;
// prefill_down's workgroups: 4 wavefronts over 512 outputs (two super-blocks),
// three workgroups per CU (168 registers per lane: the eight tiles' accumulators
// and two slices of bytes in flight).
constexpr int kDownThreads = 256, kDownWaves = kDownThreads / 64, kDownWgCols = 512;
struct DownLds {
  float h[kBlocks][4][kTileTokens][8];   // [slice][round q][token][neuron 8q + i]: gate * h * 2^-e_t
  int e[kTileTokens];                    // e_t
  // [wave][slice parity][sub-block 4hb + j of the wavefront][neuron]
  uint16_t sc[kDownWaves][2][4][kNeurons];   // 6-bit scale
  float mm[kDownWaves][2][4][kNeurons];      // dmin * m
  float d[kDownWaves][2][kNeurons];          // d
};

// v as two f16 values hi = f16(v), lo = f16(v - hi) (v - hi is exact in fp32).
__device__ __forceinline__ void split_f16(const float (&v)[8], f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    hi[j] = (_Float16)v[j];
    lo[j] = (_Float16)(v[j] - (float)hi[j]);
  }
}

__global__ __launch_bounds__(kDownThreads, 3) void prefill_down(const uint8_t* __restrict__ plan, BatchScratch S) {
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  const BatchTile T = reinterpret_cast<const BatchTile*>(plan + H.tiles_off)[blockIdx.x];
  const unsigned hidden = H.hidden, nsb = hidden / 256, nblk = H.nblk;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) DownLds L;
  const unsigned nh = nblk * kNeurons;
#pragma unroll 1
  for (unsigned th = 0; th < kTileTokens / (kDownThreads / 32); ++th) {
    // Thread (token n, j) takes neuron j of each slice of the token's
    // gate * h; the 32 threads of a token (one half wavefront) agree on e_t.
    const unsigned n = (unsigned)tid / 32 + th * (kDownThreads / 32), j = (unsigned)tid & 31;
    float v[kBlocks];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      v[i] = i < (int)nblk && n < T.ntok ? S.h[(size_t)(T.slot0 + n) * nh + kNeurons * i + j] : 0.f;
      mx = fmaxf(mx, fabsf(v[i]));
    }
#pragma unroll
    for (int o = 16; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    int E = 0;
    if (mx > 0.f) (void)frexpf(mx, &E);   // mx < 2^E
    const int e = E - 13;
#pragma unroll
    for (int i = 0; i < kBlocks; ++i)
      if (i < (int)nblk) L.h[i][j >> 3][n][j & 7] = ldexpf(v[i], -e);
    if (j == 0) L.e[n] = e;
  }
  __syncthreads();
  const unsigned sb = 2 * blockIdx.y + ((unsigned)wave >> 1), hb = (unsigned)wave & 1;
  if (sb >= nsb) return;
  const unsigned m = (unsigned)lane & 15, kq = (unsigned)lane >> 4, qa = m >> 2, qq = m & 3;
  const unsigned hn = (unsigned)lane & 31, hgg = (unsigned)lane >> 5;
  const uint64_t eoff = (uint64_t)T.expert * H.slice_bytes + 2 * H.proj + 4608 * (uint64_t)sb;
  const uint32_t shift = 4 * qq;   // the lane's output column in a unit
  uint32_t mask = 0x000F000Fu << shift;
  // Opaque to the compiler, so that (x & mask) >> shift is not rewritten as
  // (x >> shift) & 0xF000F: the AND then takes quad_nibbles' DPP read as its
  // source modifier.
  asm volatile("" : "+v"(mask));
  const uint32_t vh = 4096 + 16 * hn;                            // every lane: the header of neuron l%32
  uint32_t bad = 0, hflag = 0;   // hflag: half_bad_bits of the scale words read
  {
    // One pass over the slices for all eight tiles: tile t = 4ph + q (outputs
    // 128hb + 64ph + 16q .. +15 of the super-block) takes sub-block
    // g = 4hb + j, j = 2ph + q/2. Lane (kq, qa, qq) loads, for each half ph,
    // unit 32hb + 16ph + 4qq + qa of round kq: tile q of its quad reads the
    // unit of quad lane q. B = d h' is formed once per slice for all eight.
    const uint32_t vu = 1024 * kq + 16 * (32 * hb + 4 * qq + qa);
    struct DnBytes {
      u32x4 u[2], h;
    };
    auto load = [&](unsigned R, DnBytes& B) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<void*>(H.base[min(R, nblk - 1)] + eoff), (short)0, 4608, 0x00020000);
      B.u[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vu, 0, 0);
      B.u[1] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(vu + 256), 0, 0);
      B.h = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vh, 0, 0);
    };
    // The slice's header table (parity par): lane l decodes neuron l%32 for
    // sub-blocks j = l/32 and 2 + l/32. Returns whether the neuron's d takes
    // the direct path.
    auto table = [&](const u32x4& hd, unsigned par) {
      hflag |= half_bad_bits(hd[0]);
      const float dn = half_to_float(hd[0] & 0xffff), dmn = half_to_float(hd[0] >> 16);
      uint32_t sc0, mi0, sc1, mi1;
      q4k_scale_min(hd[1], hd[2], hd[3], 4 * hb + hgg, sc0, mi0);
      q4k_scale_min(hd[1], hd[2], hd[3], 4 * hb + 2 + hgg, sc1, mi1);
      L.sc[wave][par][hgg][hn] = (uint16_t)sc0;
      L.sc[wave][par][2 + hgg][hn] = (uint16_t)sc1;
      L.mm[wave][par][hgg][hn] = dmn * (float)mi0;
      L.mm[wave][par][2 + hgg][hn] = dmn * (float)mi1;
      if (hgg == 0) L.d[wave][par][hn] = dn;
      __builtin_amdgcn_wave_barrier();
      return fabsf(dn) < kDownDirect;
    };
    // gate * h' of the lane's token m, neurons 8kq..8kq+7 of slice R, and
    // B = d h' (times 2^-k) in two f16 parts.
    auto b_parts = [&](unsigned R, unsigned par, int k, float (&hv)[8], f16x8& bh, f16x8& bl) {
      const float4 a = *reinterpret_cast<const float4*>(&L.h[R][kq][m][0]);
      const float4 b = *reinterpret_cast<const float4*>(&L.h[R][kq][m][4]);
      const float4 d0 = *reinterpret_cast<const float4*>(&L.d[wave][par][8 * kq]);
      const float4 d1 = *reinterpret_cast<const float4*>(&L.d[wave][par][8 * kq + 4]);
      hv[0] = a.x, hv[1] = a.y, hv[2] = a.z, hv[3] = a.w, hv[4] = b.x, hv[5] = b.y, hv[6] = b.z, hv[7] = b.w;
      const float dv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = k ? ldexpf(hv[j] * dv[j], -k) : hv[j] * dv[j];
      split_f16(v, bh, bl);
    };
    // A of tile 4PH + MQ: the unit of quad lane MQ in half PH, the lane's
    // column, times sub-block 2PH + MQ/2's scales (u16 pairs of neurons
    // 8kq + 2w, 8kq + 2w + 1).
    auto a_tile = [&](const DnBytes& B, unsigned par, auto ph, auto mq) {
      constexpr int PH = decltype(ph)::value, MQ = decltype(mq)::value;
      const uint4 s4 = *reinterpret_cast<const uint4*>(&L.sc[wave][par][2 * PH + MQ / 2][8 * kq]);
      const u32x4& U = B.u[PH];
      const u32x4 aw = {scaled_u16(quad_nibbles<MQ>(U[0], mask, shift), s4.x),
                        scaled_u16(quad_nibbles<MQ>(U[1], mask, shift), s4.y),
                        scaled_u16(quad_nibbles<MQ>(U[2], mask, shift), s4.z),
                        scaled_u16(quad_nibbles<MQ>(U[3], mask, shift), s4.w)};
      return __builtin_bit_cast(f16x8, aw);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float corr[4] = {0.f, 0.f, 0.f, 0.f};   // [sub-block j] the min terms of token m, this lane's neurons
    uint32_t deferred = 0;                  // slices with a neuron's |d| >= 4 (bit R)
    auto min_terms = [&](unsigned par, const float (&hv)[8]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 m0 = *reinterpret_cast<const float4*>(&L.mm[wave][par][j][8 * kq]);
        const float4 m1 = *reinterpret_cast<const float4*>(&L.mm[wave][par][j][8 * kq + 4]);
        const float mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) corr[j] = fmaf(mv[i], hv[i], corr[j]);
      }
    };
    // Tiles 4PH..4PH+3 of one slice: A of each, times B (lo, then hi).
    auto half_tiles = [&](const DnBytes& B, unsigned par, auto ph, const f16x8& bh, const f16x8& bl) {
      constexpr int PH = decltype(ph)::value;
      auto tile = [&](auto mq) {
        constexpr int T = 4 * PH + decltype(mq)::value;
        const f16x8 a = a_tile(B, par, ph, mq);
        acc[T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, acc[T], 0, 0, 0);
        acc[T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, acc[T], 0, 0, 0);
      };
      tile(I0{});
      tile(I1{});
      tile(I2{});
      tile(I3{});
    };
    auto apply = [&](unsigned R, const DnBytes& B) {
      const unsigned par = R & 1;
      const bool direct = table(B.h, par);
      float hv[8];
      f16x8 bh, bl;
      b_parts(R, par, 0, hv, bh, bl);
      min_terms(par, hv);
      if (__builtin_expect(__ballot(!direct) != 0, 0)) {
        deferred |= 1u << R;
        return;
      }
      half_tiles(B, par, I0{}, bh, bl);
      half_tiles(B, par, I1{}, bh, bl);
    };
    DnBytes sa, sbb;
    load(0, sa);
    for (unsigned R = 0; R < nblk; R += 2) {
      load(R + 1, sbb);
      apply(R, sa);
      if (R + 1 < nblk) {
        load(R + 2, sa);
        apply(R + 1, sbb);
      }
    }
    // Deferred slices: B = d h' 2^-k with 2^k >= max |d| / 4 over the slice's
    // neurons, each product times 2^k before it joins the sum.
    for (uint32_t dm = deferred; dm; dm &= dm - 1) {
      const unsigned R = (unsigned)__builtin_ctz(dm);
      DnBytes B;
      load(R, B);
      (void)table(B.h, 0);
      float dmax = fabsf(L.d[wave][0][hn]);
      dmax = isfinite(dmax) ? dmax : 0.f;   // a non-finite d is flagged by the table
#pragma unroll
      for (int o = 16; o; o >>= 1) dmax = fmaxf(dmax, __shfl_xor(dmax, o));
      int E = 0;
      (void)frexpf(dmax, &E);   // dmax < 2^E
      const int k = max(E - 2, 0);
      float hv[8];
      f16x8 bh, bl;
      b_parts(R, 0, k, hv, bh, bl);
      // One tile at a time (its A operand alone live).
      auto scaled = [&](int t, const f16x8& a) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        f32x4 pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, z, 0, 0, 0);
        pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, pr, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] += ldexpf(pr[r], k);
      };
      scaled(0, a_tile(B, 0, I0{}, I0{}));
      scaled(1, a_tile(B, 0, I0{}, I1{}));
      scaled(2, a_tile(B, 0, I0{}, I2{}));
      scaled(3, a_tile(B, 0, I0{}, I3{}));
      scaled(4, a_tile(B, 0, I1{}, I0{}));
      scaled(5, a_tile(B, 0, I1{}, I1{}));
      scaled(6, a_tile(B, 0, I1{}, I2{}));
      scaled(7, a_tile(B, 0, I1{}, I3{}));
      __builtin_amdgcn_wave_barrier();   // the table is read before the next deferred slice writes it
    }
    // The min terms of token m over all 32 neurons: sum the four lane groups.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      corr[j] += __shfl_xor(corr[j], 16, 64);
      corr[j] += __shfl_xor(corr[j], 32, 64);
    }
    // Lane l holds C rows 4(l/16) + r (outputs 128hb + 16t + 4(l/16) + r of
    // the super-block) of token l%16: y = (C - min terms) * 2^e_t.
    if (m < T.ntok) {
      const int et = L.e[m];
      float* dst = S.part + (size_t)(T.slot0 + m) * hidden + 256 * sb + 128 * hb + 4 * kq;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float c = corr[t >> 1];
        *reinterpret_cast<float4*>(dst + 16 * t) =
            make_float4(ldexpf(acc[t][0] - c, et), ldexpf(acc[t][1] - c, et), ldexpf(acc[t][2] - c, et),
                        ldexpf(acc[t][3] - c, et));
      }
    }
  }
  if (hflag & kHalfBadBits) bad |= kErrScale;
  if (bad) flag(S.status, bad);
}

// ---------------------------------------------- prefill, row-format units
//
// The native unit (Q4_K gate/up rows, MXFP4 down [H x 32], src/native.h:9-15)
// and the shared expert of every format (Q8_0 rows, Q8_0 down [H x 32]),
// kept in the row layout the row-format decode kernel reads (row: [chunk]
// [16 B] halves, then the scales; a chunk is 64 columns). Same tiles, x'
// and h scratch as prefill_gate_up / prefill_down.
//
// Gate/up (tile, slice): wavefront w takes row-block w%4 (the gate rows of
// neurons 8rb..8rb+7, then their up rows) and chunks 2(w/4), 2(w/4)+1 of
// every super-block; one v_mfma_f32_16x16x32_f16 per 32-column sub-block,
// lane 16kg + i holding values 8kg..8kg+7 of row i: B exact in f16 (Q4_K:
// sc*q, nib_pair_sc; Q8_0: q), A = x' in two f16 parts (tokens as rows, so
// that a lane's results are its own row's). Q4_K: the super-block is scaled
// by d once and the min terms take one fp32 MFMA per four sub-blocks, as in
// prefill_gate_up; Q8_0: each sub-block's product is scaled by its row's d.
__device__ __forceinline__ uint32_t int8_pair_f16(uint32_t v, uint32_t sel) {
  // Bytes of v (signed int8) as two exact f16: 1024 + 128 + q formed in the
  // bits, less 1152.
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const uint32_t b = __builtin_amdgcn_perm(0u, v ^ 0x80808080u, sel);   // q + 128 in each 16-bit half
  const f16x2 f = __builtin_bit_cast(f16x2, b | 0x64006400u) - (f16x2){(_Float16)1152.f, (_Float16)1152.f};
  return __builtin_bit_cast(uint32_t, f);
}

template <int GU>
__global__ __launch_bounds__(kBatchThreads, 4) void prefill_gate_up_rows(const uint8_t* __restrict__ plan,
                                                                         BatchScratch S, uint32_t tile0) {
  constexpr bool kQ4 = GU == TQ4_K;
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  // XCD-contiguous runs of the (tile, slice) list, as prefill_gate_up.
  const unsigned nblk = H.nblk, per = gridDim.x / 8, b = blockIdx.x;
  const unsigned j = b < 8 * per ? (b % 8) * per + b / 8 : b, brank = j % nblk;
  const BatchTile T = reinterpret_cast<const BatchTile*>(plan + H.tiles_off)[tile0 + j / nblk];
  const BatchSlot* slots = reinterpret_cast<const BatchSlot*>(plan + H.slots_off) + T.slot0;
  const unsigned hidden = H.hidden, nsb = hidden / 256, nch = hidden / 64;
  const uint64_t proj = kQ4 ? H.proj : H.shared_proj;
  const uint8_t* slice = reinterpret_cast<const uint8_t*>(H.base[brank] + (uint64_t)T.expert * H.slice_bytes);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const unsigned rb = (unsigned)wave & 3, p = (unsigned)wave >> 2, kg = (unsigned)lane >> 4,
                 col = (unsigned)lane & 15, i = col;
  __shared__ __align__(16) GateUpLds L;
  // Q4_K rows, two super-blocks at a time: [row][half][8 chunks][16 B] (a row
  // padded to 272 bytes, so that the 16 rows a read spans fall in different
  // banks) and [row][super-block][16 B] headers; filled from registers loaded
  // one stage ahead, each row half read as one 128-byte run.
  constexpr unsigned kRowPad = 272;
  __shared__ __align__(16) uint8_t WQ[kQ4 ? 64 * kRowPad : 16];
  __shared__ __align__(16) uint4 WH[kQ4 ? 64 * 2 : 1];
  // x' staging, as prefill_gate_up: thread -> token tl, 32-byte piece c.
  const unsigned tl = (unsigned)tid >> 5, c = (unsigned)tid & 31;
  const bool live = tl < T.ntok;
  const size_t trow = (size_t)(live ? slots[tl].token : 0) * nsb;
  const uint16_t* xsrc = S.xh + trow * 512 + 16 * c;
  struct XStage {
    uint4 d[2];
    float s;
  };
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  auto load_x = [&](unsigned s, XStage& X) {
    if (live) {
      X.d[0] = *reinterpret_cast<const uint4*>(xsrc + 512 * (size_t)s);
      X.d[1] = *reinterpret_cast<const uint4*>(xsrc + 512 * (size_t)s + 8);
      if (c < 8) X.s = S.dsum[(trow + s) * 8 + c];
    }
  };
  auto store_x = [&](unsigned buf, const XStage& X) {
    uint8_t* row = &L.xh[buf][c / 16][tl][32 * (c % 16)];
    *reinterpret_cast<uint4*>(row) = X.d[0];
    *reinterpret_cast<uint4*>(row + 16) = X.d[1];
    if (c < 8) L.xs[buf][tl][c] = X.s;
  };
  // The lane's row: gate (i < 8) or up row of neuron 8rb + i%8.
  const uint8_t* row = slice + (i >> 3) * proj + (size_t)(8 * rb + (i & 7)) * (proj / kNeurons);
  // Weights of super-block s: the lane's 8-byte pieces of chunks 4s + 2p + cc
  // (Q4_K: half kg/2 of the chunk, both sub-blocks in its two nibbles; Q8_0:
  // part 2J + kg/2 of each sub-block J) and its row's scales.
  struct WStage {
    uint2 q[2][2];   // [cc][Q4_K: unused 1 | Q8_0: sub-block J]
    uint4 h;         // Q4_K: the super-block header; Q8_0: .x, .y = the scale pairs of the two chunks
  };
  auto load_w = [&](unsigned s) {
    const unsigned sc = min(s, nsb - 1);
    WStage W;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const unsigned ch = 4 * sc + 2 * p + cc;
      if (kQ4) {
        W.q[cc][0] = ld8(row + 16 * ch + 16 * nch * (kg >> 1) + 8 * (kg & 1));
        W.q[cc][1] = W.q[cc][0];
      } else {
#pragma unroll
        for (int J = 0; J < 2; ++J) W.q[cc][J] = ld8(row + 16 * nch * (2 * J + (kg >> 1)) + 16 * ch + 8 * (kg & 1));
      }
    }
    if (kQ4) {
      W.h = ld16(row + 32 * nch + 16 * sc);
    } else {
      const uint2 sp = ld8(row + 64 * nch + 4 * (4 * sc + 2 * p));
      W.h = make_uint4(sp.x, sp.y, 0u, 0u);
    }
    return W;
  };
  uint32_t bad = 0, hflag = 0;   // hflag: half_bad_bits of the scale words read
  XStage xa = {{z4, z4}, 0.f}, xb = {{z4, z4}, 0.f};
  load_x(0, xa);
  store_x(0, xa);
  if (1 < nsb) load_x(1, xa);
  __syncthreads();
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  f32x4 cmin = {0.f, 0.f, 0.f, 0.f};
  // Super-block s: W holds its weights, cur holds x' of s+1 (stored at the
  // end), s+2 is loaded into nxt.
  auto step = [&](unsigned s, const WStage& W, XStage& cur, XStage& nxt) {
    const unsigned buf = s & 1;
    if (s + 2 < nsb) load_x(s + 2, nxt);
    f32x4 c_hi = {0.f, 0.f, 0.f, 0.f}, c_lo = {0.f, 0.f, 0.f, 0.f};
    f16x2 scs[2][2] = {};
    if (kQ4) {
      hflag |= half_bad_bits(W.h.x);
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int J = 0; J < 2; ++J) {
          uint32_t sc, mi;
          q4k_scale_min(W.h.y, W.h.z, W.h.w, 4 * p + 2 * cc + J, sc, mi);
          scs[cc][J] = f16_pair(sc);
        }
    }
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        const unsigned sub = 4 * p + 2 * cc + J;   // sub-block of the super-block
        u32x4 aw;
        if (kQ4) {
          const uint32_t w0 = J ? nib_hi(W.q[cc][0].x) : nib_lo(W.q[cc][0].x);
          const uint32_t w1 = J ? nib_hi(W.q[cc][0].y) : nib_lo(W.q[cc][0].y);
          aw = u32x4{nib_pair_sc<false>(w0, scs[cc][J]), nib_pair_sc<true>(w0, scs[cc][J]),
                     nib_pair_sc<false>(w1, scs[cc][J]), nib_pair_sc<true>(w1, scs[cc][J])};
        } else {
          const uint2 q = W.q[cc][J];
          aw = u32x4{int8_pair_f16(q.x, 0x0c010c00u), int8_pair_f16(q.x, 0x0c030c02u), int8_pair_f16(q.y, 0x0c010c00u),
                     int8_pair_f16(q.y, 0x0c030c02u)};
        }
        const f16x8 a = __builtin_bit_cast(f16x8, aw);
        const uint8_t* xb8 = &L.xh[buf][0][col][2 * (32 * sub + 8 * kg)];
        const uint4 bh = *reinterpret_cast<const uint4*>(xb8);
        const uint4 bl = *reinterpret_cast<const uint4*>(xb8 + kTileTokens * kXhRow);
        if (kQ4) {
          c_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bh), a, c_hi, 0, 0, 0);
          c_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bl), a, c_lo, 0, 0, 0);
        } else {
          // The row's Q8_0 scale of this sub-block (scales of chunk 4s+2p+cc,
          // half J): the lane's results are all of its own row.
          const uint32_t sp = cc ? W.h.y : W.h.x;
          const uint32_t hb = J ? sp >> 16 : sp & 0xffffu;
          if (J == 0) hflag |= half_bad_bits(sp);   // both halves: this sub-block's scale and the next one's
          const float d = half_to_float(hb);
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          const f32x4 ph = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bh), a, z, 0, 0, 0);
          const f32x4 pl = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bl), a, z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, ph[r] + pl[r], acc[r]);
        }
      }
    if (kQ4) {
      const float d = half_to_float(W.h.x & 0xffff);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, c_hi[r] + c_lo[r], acc[r]);
      // Min terms of sub-blocks 4p..4p+3: B = -dmin * m of (4p + kg, row i).
      uint32_t sc, mi;
      q4k_scale_min(W.h.y, W.h.z, W.h.w, 4 * p + kg, sc, mi);
      cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(L.xs[buf][col][4 * p + kg], -half_to_float(W.h.x >> 16) * (float)mi,
                                                  cmin, 0, 0, 0);
    }
  };
  auto finish = [&](unsigned s, const XStage& cur) {
    if (s + 1 < nsb) store_x((s & 1) ^ 1, cur);
    __syncthreads();
  };
  if constexpr (kQ4) {
    // Thread -> two 16-byte pieces of quants (piece tid + 512j: row pc/16,
    // half (pc/8)%2, super-block (pc/4)%2 of the stage, chunk pc%4) and, for
    // tid < 128, one header (row tid/2, super-block tid%2).
    const unsigned rowb = (unsigned)(proj / kNeurons), half = 16 * nch;
    auto grow = [&](unsigned r) {   // row r of the slice: gate (r%16 < 8) or up of neuron 8(r/16) + r%8
      return slice + ((r & 15) >> 3) * proj + (size_t)(8 * (r >> 4) + (r & 7)) * rowb;
    };
    uint4 gq[2], gh = make_uint4(0u, 0u, 0u, 0u);
    auto load_stage = [&](unsigned s0) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const unsigned pc = (unsigned)tid + 512 * jj, r = pc >> 4, hf = (pc >> 3) & 1;
        const unsigned sb = min(s0 + ((pc >> 2) & 1), nsb - 1);
        gq[jj] = ld16(grow(r) + hf * half + 16 * (4 * sb + (pc & 3)));
      }
      if (tid < 128) gh = ld16(grow((unsigned)tid >> 1) + 2 * half + 16 * min(s0 + ((unsigned)tid & 1), nsb - 1));
    };
    auto store_stage = [&]() {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const unsigned pc = (unsigned)tid + 512 * jj, r = pc >> 4, hf = (pc >> 3) & 1;
        *reinterpret_cast<uint4*>(&WQ[kRowPad * r + 128 * hf + 16 * (pc & 7)]) = gq[jj];
      }
      if (tid < 128) WH[tid] = gh;
    };
    // The lane's weights of super-block sbl of the stage, from LDS.
    const unsigned lrow = 16 * rb + i;
    auto lds_w = [&](unsigned sbl) {
      WStage W;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        W.q[cc][0] = *reinterpret_cast<const uint2*>(
            &WQ[kRowPad * lrow + 128 * (kg >> 1) + 16 * (4 * sbl + 2 * p + cc) + 8 * (kg & 1)]);
        W.q[cc][1] = W.q[cc][0];
      }
      W.h = WH[2 * lrow + sbl];
      return W;
    };
    load_stage(0);
    for (unsigned s0 = 0; s0 < nsb; s0 += 2) {
      store_stage();
      if (s0 + 2 < nsb) load_stage(s0 + 2);
      __syncthreads();   // the stage's weights are in LDS
      {
        XStage& cur = (s0 & 1) ? xb : xa;
        XStage& nxt = (s0 & 1) ? xa : xb;
        step(s0, lds_w(0), cur, nxt);
        finish(s0, cur);
      }
      if (s0 + 1 < nsb) {
        XStage& cur = ((s0 + 1) & 1) ? xb : xa;
        XStage& nxt = ((s0 + 1) & 1) ? xa : xb;
        step(s0 + 1, lds_w(1), cur, nxt);
        finish(s0 + 1, cur);
      }
    }
  } else {
    // Rotating register sets, three super-blocks ahead, unrolled by six so
    // that no set is copied while its loads are in flight (as
    // prefill_gate_up).
    WStage wa = load_w(0), wb = load_w(1), wc = load_w(2);
    auto go = [&](unsigned s, WStage& W, XStage& cur, XStage& nxt) {
      step(s, W, cur, nxt);
      W = load_w(s + 3);
      finish(s, cur);
    };
    for (unsigned s = 0; s < nsb; s += 6) {
      go(s, wa, xa, xb);
      if (s + 1 < nsb) go(s + 1, wb, xb, xa);
      if (s + 2 < nsb) go(s + 2, wc, xa, xb);
      if (s + 3 < nsb) go(s + 3, wa, xb, xa);
      if (s + 4 < nsb) go(s + 4, wb, xa, xb);
      if (s + 5 < nsb) go(s + 5, wc, xb, xa);
    }
  }
  // Lane (kg, col) holds tokens 4kg..4kg+3 of row col.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    L.main[wave][col][4 * kg + r] = acc[r];
    L.mins[wave][col][4 * kg + r] = cmin[r];
  }
  __syncthreads();
  {
    const unsigned trb = (unsigned)tid >> 7, ni = ((unsigned)tid >> 4) & 7, n = (unsigned)tid & 15;
    if (n < T.ntok) {
      const float sx = S.dscale[slots[n].token];
      const float a = ((L.main[trb][ni][n] + L.mins[trb][ni][n]) + (L.main[trb + 4][ni][n] + L.mins[trb + 4][ni][n])) * sx;
      const float u = ((L.main[trb][8 + ni][n] + L.mins[trb][8 + ni][n]) +
                       (L.main[trb + 4][8 + ni][n] + L.mins[trb + 4][8 + ni][n])) * sx;
      uint32_t hb = 0;
      const float h = slots[n].gate * silu_mul_f32(a, u, hb);
      bad |= hb;
      S.h[(size_t)(T.slot0 + n) * (nblk * kNeurons) + kNeurons * brank + 8 * trb + ni] = h;
    }
  }
  if (hflag & kHalfBadBits) bad |= kErrScale;
  if (bad) flag(S.status, bad);
}

// Down (tile, 128 kT outputs) of row-format units: output o's 32 neurons as
// one record (MXFP4: 16 code bytes at 16o, neuron j in the low nibble of byte
// j, 16 + j in its high nibble, E8M0 exponent at 16H + o; Q8_0: 16 int8 at
// 16o, 16 more at 16H + 16o, the fp16 d at 32H + 2o). Wavefront w takes the
// kT 16-output tiles from output 16 kT w of the workgroup's; per slice and
// tile, v_mfma_f32_16x16x32_bf16 over the 32 neurons: lane group kq takes
// neurons 4kq + i and 16 + 4kq + i (i = 0..3), byte i of the record's dword
// kq, the one dword of the record that the lane loads. B = h of those neurons
// for the tile's tokens in three bf16 parts that sum to it exactly (three
// products), split once per workgroup into LDS.
// MXFP4: A = code * 2^(e-127) of the lane's output row by
// v_cvt_scalef32_pk_bf16_fp4, exact (a code has two significant bits, and the
// product is a normal bf16 for e = 2..254), so the products add straight into
// the tile's accumulators over the slices. Exponents 253..255 pass the
// overflow screen of src/native.c:23-27 first. A slice in which some lane
// holds an exponent below 64 (weights below 2^-63, which no real unit has)
// is deferred to the end and taken as the exact codes with each row's
// 2^(e-127) applied after the product, as fp32 scaling, so that no product
// of the matrix cores comes near the subnormal range.
// Q8_0: A = the int8 of q0 and q1 exactly; each slice's product is scaled per
// output row by d before it joins the sum over slices.
constexpr int kDownRowsTilesMx = 8;   // tiles per wavefront, MXFP4 (routed)
constexpr uint32_t kMxDirect = 64;    // smallest exponent scaled inside the products
constexpr int kDownRowsTilesQ8 = 4;   // Q8_0 (the shared expert): twice the workgroups
template <int DN>
constexpr unsigned down_rows_cols() {
  return 128u * (DN == TMXFP4 ? kDownRowsTilesMx : kDownRowsTilesQ8);
}
struct DownRowsLds {
  bf16x8 b[kBlocks][3][64];   // [slice][part][lane 16kq + token m]: k-slots 2i, 2i+1 = neurons 4kq + i, 16 + 4kq + i
};
// The Q8_0 instantiation holds twice the record bytes per tile and takes two
// wavefronts per SIMD instead of four.
template <int DN>
__global__ __launch_bounds__(kBatchThreads, DN == TMXFP4 ? 4 : 2) void prefill_down_rows(const uint8_t* __restrict__ plan,
                                                                                          BatchScratch S,
                                                                                          uint32_t tile0) {
  constexpr bool kMx = DN == TMXFP4;
  constexpr int kT = kMx ? kDownRowsTilesMx : kDownRowsTilesQ8;
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  const BatchTile T = reinterpret_cast<const BatchTile*>(plan + H.tiles_off)[tile0 + blockIdx.x];
  const unsigned hidden = H.hidden, nblk = H.nblk;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) DownRowsLds L;
  const unsigned nh = nblk * kNeurons;
  // Item (slice R, lane 16kq + n): token n's gate * h of neurons 4kq..4kq+3
  // and 16 + 4kq..+3, interleaved into the lane's k-slots, in three parts.
  for (unsigned k = (unsigned)tid; k < nblk * 64; k += kBatchThreads) {
    const unsigned R = k >> 6, ln = k & 63, kq = ln >> 4, n = ln & 15;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a;
    if (n < T.ntok) {
      const float* src = S.h + (size_t)(T.slot0 + n) * nh + kNeurons * R + 4 * kq;
      a = *reinterpret_cast<const float4*>(src);
      c = *reinterpret_cast<const float4*>(src + 16);
    }
    const float hv[8] = {a.x, c.x, a.y, c.y, a.z, c.z, a.w, c.w};
    bf16x8 b1, b2, b3;
    split_bf16(hv, b1, b2, b3);
    L.b[R][0][ln] = b1;
    L.b[R][1][ln] = b2;
    L.b[R][2][ln] = b3;
  }
  __syncthreads();
  const unsigned o0 = down_rows_cols<DN>() * blockIdx.y + 16 * kT * (unsigned)wave;
  if (o0 >= hidden) return;
  const unsigned m = (unsigned)lane & 15, kq = (unsigned)lane >> 4;
  const uint64_t proj = kMx ? H.proj : H.shared_proj;
  const uint64_t eoff = (uint64_t)T.expert * H.slice_bytes + 2 * proj;
  const int nrec = (int)((kMx ? 17u : 34u) * hidden);   // the down's bytes
  const uint32_t vw = 16 * (o0 + m) + 4 * kq;           // dword kq of output o0 + m (tile t: + 256t)
  const uint32_t ve = 16 * hidden + o0 + 4 * (lane & 31);   // MXFP4: dword l%32 of the wavefront's 128 exponents
  const uint32_t vr = 16 * hidden + o0 + 4 * kq;        // MXFP4: exponents of the lane's C rows (+ 16t)
  const uint32_t vs = 32 * hidden + 2 * (o0 + 4 * kq);  // Q8_0: d of the lane's C rows (+ 32t)
  uint32_t bad = 0;
  // A slice's bytes, two slices ahead in three register sets (the loop is
  // unrolled by three so that no set is copied while its loads are in
  // flight). MXFP4: one dword of exponents per lane; lane 4t + m/4 holds
  // those of tile t's outputs 16t + 4(m/4) .. +3.
  struct MxSlice {
    uint32_t w[kT], e32;
  };
  struct Q8Slice {
    uint32_t q0[kT], q1[kT];
    u32x2 s[kT];
  };
  using SliceBytes = typename std::conditional<kMx, MxSlice, Q8Slice>::type;
  auto load_slice = [&](unsigned R, SliceBytes& B) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(H.base[min(R, nblk - 1)] + eoff), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      if constexpr (kMx) {
        B.w[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(vw + 256 * t), 0, 0);
      } else {
        B.q0[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(vw + 256 * t), 0, 0);
        B.q1[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(16 * hidden + vw + 256 * t), 0, 0);
        B.s[t] = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(vs + 32 * t), 0, 0);
      }
    }
    if constexpr (kMx) B.e32 = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)ve, 0, 0);
  };
  f32x4 acc[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  uint32_t deferred = 0;   // MXFP4: slices in which some lane holds e < kMxDirect (bit R)
  auto apply = [&](unsigned R, const SliceBytes& B) {
    const bf16x8 b1 = L.b[R][0][lane], b2 = L.b[R][1][lane], b3 = L.b[R][2][lane];
    if constexpr (kMx) {
      uint32_t ev[kT];   // the exponent of the lane's output in each tile
#pragma unroll
      for (int t = 0; t < kT; ++t)
        ev[t] = ((uint32_t)__shfl((int)B.e32, (int)(4 * t + (m >> 2))) >> (8 * (m & 3))) & 0xffu;
      uint32_t lo = ev[0], hi = ev[0];
#pragma unroll
      for (int t = 1; t < kT; ++t) {
        lo = min(lo, ev[t]);
        hi = max(hi, ev[t]);
      }
      if (__builtin_expect(__ballot(hi >= 253u) != 0, 0)) {
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          // The record's screen: its four dwords lie in lanes m, m+16, m+32, m+48.
          const uint32_t w = B.w[t], e = ev[t];
          uint32_t ge2 = w & 0x44444444u, ge4 = w & (w >> 1) & 0x22222222u;
          ge2 |= (uint32_t)__shfl_xor((int)ge2, 16);
          ge2 |= (uint32_t)__shfl_xor((int)ge2, 32);
          ge4 |= (uint32_t)__shfl_xor((int)ge4, 16);
          ge4 |= (uint32_t)__shfl_xor((int)ge4, 32);
          if (kq == 0 && (e == 255u || (e == 254u && ge2 != 0u) || (e == 253u && ge4 != 0u))) bad |= kErrScale;
        }
      }
      if (__builtin_expect(__ballot(lo < kMxDirect) != 0, 0)) {
        deferred |= 1u << R;   // after the loop, on the exact codes
      } else {
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          // 2^(e-127), e = 64..255 (a block at 253..255 that overflows is flagged above).
          const float sc = __uint_as_float(ev[t] << 23);
          const u32x4 aw = {
              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(B.w[t], sc, 0)),
              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(B.w[t], sc, 1)),
              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(B.w[t], sc, 2)),
              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(B.w[t], sc, 3))};
          const bf16x8 av = __builtin_bit_cast(bf16x8, aw);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b3, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b2, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b1, acc[t], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        u32x4 aw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // int8 -> fp32 exactly; the bf16 is its upper half.
          const uint32_t lo = __float_as_uint((float)(int8_t)(B.q0[t] >> (8 * i)));
          const uint32_t hi = __float_as_uint((float)(int8_t)(B.q1[t] >> (8 * i)));
          aw[i] = (lo >> 16) | (hi & 0xffff0000u);
        }
        const uint32_t hs[4] = {B.s[t].x & 0xffffu, B.s[t].x >> 16, B.s[t].y & 0xffffu, B.s[t].y >> 16};
        float sc[4];   // d of the lane's C rows: outputs o0 + 16t + 4kq .. +3
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (half_bad(hs[r])) bad |= kErrScale;
          sc[r] = half_to_float(hs[r]);
        }
        const bf16x8 av = __builtin_bit_cast(bf16x8, aw);
        f32x4 pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b3, z, 0, 0, 0);
        pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b2, pr, 0, 0, 0);
        pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b1, pr, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(sc[r], pr[r], acc[t][r]);
      }
    }
  };
  SliceBytes sa, sb, sc;
  load_slice(0, sa);
  load_slice(1, sb);
  for (unsigned R = 0; R < nblk; R += 3) {
    load_slice(R + 2, sc);
    apply(R, sa);
    if (R + 1 < nblk) {
      load_slice(R + 3, sa);
      apply(R + 1, sb);
    }
    if (R + 2 < nblk) {
      load_slice(R + 4, sb);
      apply(R + 2, sc);
    }
  }
  // The deferred MXFP4 slices: the exact codes, then each C row's 2^(e-127)
  // (lane 16kq + m reads the exponents of outputs o0 + 16t + 4kq .. +3).
  // Added after the other slices: a float sum in another order.
  for (uint32_t dm = deferred; dm; dm &= dm - 1) {
    const unsigned R = (unsigned)__builtin_ctz(dm);
    const bf16x8 b1 = L.b[R][0][lane], b2 = L.b[R][1][lane], b3 = L.b[R][2][lane];
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(H.base[R] + eoff), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(vw + 256 * t), 0, 0);
      const uint32_t er = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(vr + 16 * t), 0, 0);
      const u32x4 aw = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3))};
      const bf16x8 av = __builtin_bit_cast(bf16x8, aw);
      f32x4 pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b3, z, 0, 0, 0);
      pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b2, pr, 0, 0, 0);
      pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b1, pr, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(e8m0((er >> (8 * r)) & 0xffu), pr[r], acc[t][r]);
    }
  }
  // Lane l holds C rows 4(l/16) + r (outputs o0 + 16t + 4kq + r) of token m.
  if (m < T.ntok) {
    float* dst = S.part + (size_t)(T.slot0 + m) * hidden + o0 + 4 * kq;
#pragma unroll
    for (int t = 0; t < kT; ++t)
      *reinterpret_cast<float4*>(dst + 16 * t) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
  }
  if (bad) flag(S.status, bad);
}

// Token t's outputs 1024 by..+1023: its 10 expert partials in routing order,
// then the shared expert's if it has one, summed in fp64, narrowed to fp32
// with the reference's overflow rule.
__global__ __launch_bounds__(256) void prefill_reduce(const uint8_t* __restrict__ plan, BatchScratch S) {
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(plan);
  const unsigned t = blockIdx.x, hidden = H.hidden, c = kDownCols * blockIdx.y + 4 * threadIdx.x;
  if (c >= hidden) return;
  const uint32_t* ts = reinterpret_cast<const uint32_t*>(plan + H.tokslot_off) + 11 * (size_t)t;
  const int ne = ts[10] != kNoSlot ? 11 : 10;
  double a[4] = {0.0, 0.0, 0.0, 0.0};
  for (int e = 0; e < ne; ++e) {
    const float4 v = *reinterpret_cast<const float4*>(S.part + (size_t)ts[e] * hidden + c);
    a[0] += v.x;
    a[1] += v.y;
    a[2] += v.z;
    a[3] += v.w;
  }
  float y[4];
  uint32_t bad = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (!isfinite(a[j]) || fabs(a[j]) > (double)FLT_MAX) bad = kErrRange;
    y[j] = (float)a[j];
  }
  *reinterpret_cast<float4*>(S.y + (size_t)t * hidden + c) = make_float4(y[0], y[1], y[2], y[3]);
  if (bad) flag(S.status, bad);
}

// Debug: decode re-tiled gate/up row(s) with the hot path's decoder.
__global__ void debug_decode_rows(uint8_t type, const uint8_t* row, uint32_t n, float* out, uint32_t* status) {
  int c = threadIdx.x;
  uint32_t nch = n / 64;
  if (c >= (int)nch) return;
  float w[64];
  if (!decode_lane(type, row, nch, c, w)) atomicOr(status, kErrScale);
  for (int j = 0; j < 64; ++j) {
    // lane chunk column -> row column
    uint32_t col;
    if (type == TQ4_K) col = 64 * c + j;                 // chunk columns in order
    else col = 64 * c + j;                               // two 32-blocks in order
    out[col] = w[j];
  }
}

__global__ void debug_decode_down(uint8_t dn, const uint8_t* down, uint32_t hidden, float* out, uint32_t* status) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (dn == TQ4_KT) {
    // thread = (super-block, lane)
    uint32_t sb = i / 64, l = i % 64;
    if (sb >= hidden / 256) return;
    float w[128];
    if (!decode_down_q4kt(down, sb, (int)l, w)) atomicOr(status, kErrScale);
    for (int n = 0; n < 32; ++n)
      for (int cc = 0; cc < 4; ++cc) out[(size_t)(256 * sb + 4 * l + cc) * 32 + n] = w[4 * n + cc];
    return;
  }
  if (i >= hidden) return;
  float w[32];
  if (!decode_down_row(dn, down, hidden, i, w)) atomicOr(status, kErrScale);
  for (int n = 0; n < 32; ++n) out[(size_t)i * 32 + n] = w[n];
}

__global__ void debug_retile_row(SliceShape s, const uint8_t* in, uint8_t* outb, uint32_t bytes) {
  for (uint32_t o = threadIdx.x; o < bytes; o += blockDim.x) outb[o] = in[gu_source((uint8_t)s.gu, s.hidden / 64, o)];
}

__global__ void debug_retile_down(uint8_t dn, uint32_t hidden, const uint8_t* in, uint8_t* outb, uint32_t bytes) {
  for (uint32_t o = threadIdx.x; o < bytes; o += blockDim.x)
    outb[o] = dn == TQ4_KT ? q4kt_byte(in, 0u, hidden, o) : in[down_source(dn, hidden, o)];
}

__global__ void debug_quantize(float* x, uint32_t groups) {
  uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g < groups) q8_group(x + 64 * g, 64);
}

// The register form: one 64-value group per thread through q8_regs64.
__global__ void debug_quantize_regs(float* x, uint32_t groups) {
  uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  float4 v[16];
  float4* p = reinterpret_cast<float4*>(x + 64 * (size_t)g);
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = p[i];
  q8_regs64(v);
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = v[i];
}

__global__ void debug_quantize32(float* x, uint32_t groups) {
  uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g < groups) q8_group(x + 32 * g, 32);
}

// quantize8 of one token's x (group 256) through the q8_256 staging of the
// row-format kernel, read back from LDS: each value's code, d per 256 and
// the int16 sum per 32 (hidden <= kMaxHidden, a multiple of 256).
__global__ __launch_bounds__(kDecodeThreads) void debug_quantize8_x(const float* x, uint32_t hidden, int8_t* q,
                                                                    float* d, int16_t* s) {
  __shared__ __align__(16) RowsLds L;
  const unsigned tid = threadIdx.x, nsub = hidden / 32, sb = tid >> 2, k = tid & 3;
  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  if (sb < nsub) {
    const float4* xs = reinterpret_cast<const float4*>(x + 32 * sb + 8 * k);
    xv[0] = xs[0];
    xv[1] = xs[1];
  }
  uint32_t bad = 0;
  stage_x_q256(xv, nsub, L, bad);
  __syncthreads();
  if (sb >= nsub) return;
  const uint2 w = *reinterpret_cast<const uint2*>(&L.xl[0][sb & 1][k >> 1][sb >> 1][2 * (k & 1)]);
#pragma unroll
  for (int i = 0; i < 8; ++i) q[32 * sb + 8 * k + i] = (int8_t)((i < 4 ? w.x : w.y) >> (8 * (i & 3)));
  if (k == 0) {
    const float dg = L.xw[sb][0];
    if (sb % 8 == 0) d[sb / 8] = dg;
    s[sb] = dg == 0.f ? (int16_t)0 : (int16_t)(L.xsd[sb] / (double)dg);   // exact: the sum times d
  }
}

// fr_q8_activation as the ref-q8 decode kernels apply it, read back from
// their LDS: x of one token (up to 4096 values) staged by stage_x_q8 into
// decode_q8_kernel's layout (form 0) or decode_rows_q8_kernel's lane-major
// layout (form 1), each value rebuilt from its two digits as s*k + u*r, with
// the staged exact sum of each 32-value sub-block; or 32 h values through
// quantize_h32 (form 2). status gets the staging's error bits.
__global__ __launch_bounds__(kDecodeThreads) void debug_quantize_staged(const float* x, uint32_t n, uint32_t form,
                                                                       float* out, double* sums, uint32_t* status) {
  __shared__ __align__(16) DecodeQ8Lds L;
  __shared__ __align__(16) RowsLds R;
  const unsigned tid = threadIdx.x, lane = tid & 63;
  uint32_t bad = 0;
  if (form == 2) {
    if (tid < 64) {
      float* hs = L.h[0];
      if (lane < 32) hs[lane] = x[lane];
      __builtin_amdgcn_wave_barrier();
      quantize_h32(hs, (int)lane);
      if (lane < 32) out[lane] = hs[lane];
    }
    return;
  }
  const unsigned nsub = n / 32, sb = tid >> 2, q = tid & 3;
  float4 xv[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  if (sb < nsub) {
    const float4* xs = reinterpret_cast<const float4*>(x + 32 * sb + 8 * q);
    xv[0] = xs[0];
    xv[1] = xs[1];
  }
  if (form == 0) stage_x_q8(xv, 0, nsub, L, bad);
  else stage_x_q8<RowsLds, true>(xv, 0, nsub, R, bad);
  __syncthreads();
  if (bad) flag(status, bad);
  if (sb >= nsub) return;
  uint2 k, r;
  float ws, wu;
  double sum;
  if (form == 0) {
    k = *reinterpret_cast<const uint2*>(&L.xd[0][0][sb][8 * q]);
    r = *reinterpret_cast<const uint2*>(&L.xd[0][1][sb][8 * q]);
    ws = L.xw[0][sb][0];
    wu = L.xw[0][sb][1];
    sum = L.xs[0][sb];
  } else {
    k = *reinterpret_cast<const uint2*>(&R.xl[0][sb & 1][q >> 1][sb >> 1][2 * (q & 1)]);
    r = *reinterpret_cast<const uint2*>(&R.xl[1][sb & 1][q >> 1][sb >> 1][2 * (q & 1)]);
    ws = R.xw[sb][0];
    wu = R.xw[sb][1];
    sum = R.xsd[sb];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int kd = (int8_t)((i < 4 ? k.x : k.y) >> (8 * (i & 3)));
    const int rd = (int8_t)((i < 4 ? r.x : r.y) >> (8 * (i & 3)));
    out[32 * sb + 8 * q + i] = (float)((double)kd * (double)ws + (double)rd * (double)wu);
  }
  if (q == 0) sums[sb] = sum;
}

// quantize8 of 32 h values (group 32) through the q8_256 h quantizer.
__global__ __launch_bounds__(64) void debug_quantize8_h(const float* h, int8_t* q, float* d) {
  __shared__ float hs[32];
  __shared__ float md;
  const int lane = threadIdx.x;
  if (lane < 32) hs[lane] = h[lane];
  __syncthreads();
  quantize_h32_q256(hs, &md, lane);
  __syncthreads();
  if (lane < 32) q[lane] = (int8_t)hs[lane];
  if (lane == 0) *d = md;
}

// ================================================================ host

// ------------------------------------------------------ static scratch
//
// fr_hip_launch_static's scratch, for callers that cannot allocate: the
// decode kernels' error word (in a 256-byte first block), then the
// partials of up to kStaticUnits items ([position block][item][16]). Each
// GPU the library runs on holds it (4.2 MB) until the process ends. Host
// code reaches it only through the address hipGetSymbolAddress returns.
constexpr uint32_t kStaticUnits = 256;   // one token's items: 11 experts x 20 blocks, or split units of fewer blocks
constexpr size_t kStaticHead = 64;       // floats before the partials (the error word, padded)
constexpr size_t kStaticFloats = kStaticHead + (size_t)(kMaxHidden / 16) * kStaticUnits * 16;
static __device__ __align__(256) float scratch[kStaticFloats];
static_assert(kDecodeUnitsPerToken <= (int)kStaticUnits, "a token's units fit the static scratch");

// ------------------------------------------------------------ stream probe
//
// Measurement only: the achievable read bandwidth of a set of byte ranges,
// in the spirit of backends/metal.m:265-270 and tools/avx2-probe.c:12-30.
// Workgroup b reads pieces[b] = (device address, length) with 16-byte raw
// buffer loads, each thread keeping DEPTH loads in flight (a load past the
// piece returns zero without a memory access), and each wavefront stores the
// XOR of what it read so that the loads stay live.
template <int DEPTH>
__global__ __launch_bounds__(1024) void stream_probe(const uint64_t* __restrict__ pieces, uint32_t* __restrict__ sink) {
  const uint64_t addr = pieces[2 * blockIdx.x], len = pieces[2 * blockIdx.x + 1];
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(addr), (short)0, (int)len, 0x00020000);
  const uint32_t step = 16u * blockDim.x;
  uint32_t acc = 0;
  for (uint32_t off = 16u * threadIdx.x; off < (uint32_t)len; off += DEPTH * step) {
    u32x4 v[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) v[d] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + d * step), 0, 0);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
  if ((threadIdx.x & 63) == 0) sink[16 * blockIdx.x + (threadIdx.x >> 6)] = acc;
}

struct Layout {
  uint32_t hidden, format, gu, dn, shared_gu, shared_dn;
  uint64_t proj, down, slice, shared_proj, shared_slice, layer, block;
};

uint64_t row_bytes(uint32_t type, uint32_t n) {
  switch (type) {
    case TQ4_K:
    case TQ4_KM: return (uint64_t)n / 256 * 144;
    case TMXFP4: return (uint64_t)n / 32 * 17;
    case TQ8_0: return (uint64_t)n / 32 * 34;
    case TQ4_0: return (uint64_t)n / 32 * 18;
    default: return 0;
  }
}

bool layout_of(uint32_t hidden, uint32_t format, Layout& l) {
  if (!hidden || hidden > (uint32_t)kMaxHidden || hidden % kCols) return false;
  memset(&l, 0, sizeof(l));
  l.hidden = hidden;
  l.format = format;
  switch (format) {
    case FR_HIP_FMT_LEGACY: l.gu = TQ4_0; l.dn = TQ4_0; break;
    case FR_HIP_FMT_NATIVE: l.gu = TQ4_K; l.dn = TMXFP4; break;
    case FR_HIP_FMT_Q4KT: l.gu = TQ4_KM; l.dn = TQ4_KT; break;
    case FR_HIP_FMT_Q8: l.gu = TQ8_0; l.dn = TQ8_0; break;
    case FR_HIP_FMT_MXFP4: l.gu = TMXFP4; l.dn = TMXFP4; break;
    default: return false;
  }
  l.proj = kNeurons * row_bytes(l.gu, hidden);
  l.down = l.dn == TQ4_KT ? kNeurons * row_bytes(TQ4_K, hidden) : (uint64_t)hidden * row_bytes(l.dn, kNeurons);
  l.slice = 2 * l.proj + l.down;
  if (format == FR_HIP_FMT_LEGACY) {
    l.shared_gu = l.shared_dn = TQ4_0;
    l.shared_proj = l.proj;
    l.shared_slice = l.slice;
  } else {
    l.shared_gu = l.shared_dn = TQ8_0;
    l.shared_proj = kNeurons * row_bytes(TQ8_0, hidden);
    l.shared_slice = 3 * l.shared_proj;
  }
  l.layer = (uint64_t)kRouted * l.slice + l.shared_slice;
  l.block = (uint64_t)kLayers * l.layer;
  return true;
}

SliceShape shape_of(const Layout& l, bool shared) {
  SliceShape s;
  s.hidden = l.hidden;
  s.gu = shared ? l.shared_gu : l.gu;
  s.dn = shared ? l.shared_dn : l.dn;
  s.proj = (uint32_t)(shared ? l.shared_proj : l.proj);
  s.down = (uint32_t)(shared ? l.shared_proj : l.down);
  s.slice = (uint32_t)(shared ? l.shared_slice : l.slice);
  return s;
}

struct Engine {
  int device = -1;
  unsigned cus = 0;               // compute units: bound on co-resident decode workgroups
  hipStream_t stream = nullptr;
  uint8_t* block[kBlocks] = {};
  Layout lay[kBlocks];
  uint32_t layers[kBlocks] = {};  // resident layers [0, layers) of each block
  uint32_t* done = nullptr;       // [2][kMaxPairs]
  uint32_t* fin = nullptr;        // [2][kMaxRanges]
  float* hbuf = nullptr;          // [kMaxPairs][8][32]
  double* partial = nullptr;
  size_t partial_bytes = 0;
  uint32_t* out = nullptr;        // [2][out_words]
  uint32_t out_words = 0;
  float* wgpart = nullptr;        // [kMaxDecodeItems][kMaxHidden] of float, or of double for ref-q8 plans
  uint32_t* bar = nullptr;        // [2]
  float* static_scratch = nullptr;   // device address of `scratch` on this engine's device
  // fr_hip_run's decode-path outputs in mapped pinned host memory (the host
  // pointer and the device's view of it): y [8][4096] and one status word
  // per decode_reduce workgroup [8][256]; and decode_kernel's error word.
  float* hy_host = nullptr;
  float* hy_dev = nullptr;
  uint32_t* hstat_host = nullptr;
  uint32_t* hstat_dev = nullptr;
  uint32_t* hdstat = nullptr;
  // Read once at open (environment), not per run: the down-phase group
  // bytes of layer_kernel and the switch that routes requests past the
  // decode kernels (fr_hip_route changes it later).
  uint32_t group_bytes = 49152;
  bool no_decode = false;
  bool no_burst = false;          // bursts of all-Q4_K units one unit per (token, pair) on decode_kernel
  bool force_burst = false;       // every such burst on decode_burst_kernel, whatever its expert sharing
  uint8_t* plan_dev = nullptr;
  uint8_t* plan_host = nullptr;   // pinned, mapped
  const uint4* plan_mapped = nullptr;   // the device's view of plan_host
  size_t plan_cap = 0;
  uint32_t* out_host = nullptr;   // pinned: status, pad x3, y
  uint8_t* staging = nullptr;     // device staging for uploads
  size_t staging_bytes = 0;
  uint32_t parity = 0;
  uint32_t last_parity = 0;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  fr_hip_sample sample = {};
  // fr_hip_run's phase sample: the last call's phases (ns), the calls
  // sampled, and events around its launches while phase_events is set.
  double phase[FR_HIP_PHASES] = {};
  uint64_t phase_runs = 0;
  bool phase_events = false;
  hipEvent_t pev0 = nullptr, pev1 = nullptr;
  // Launch timing (fr_hip_timing): events before, between and after the
  // kernels of each launch, for the first `timed_cap` launches.
  hipEvent_t* tev = nullptr;
  unsigned timed_cap = 0, timed = 0;
  bool timing = false;
  // Prefill path: scratch (grown on demand), status word, plan buffers.
  float* bh = nullptr;
  float* bpart = nullptr;
  float* by = nullptr;
  uint8_t* bdig = nullptr;            // x' parts, then sub-block sums, then 2^e
  size_t bh_bytes = 0, bpart_bytes = 0, by_bytes = 0, bdig_bytes = 0;
  uint32_t* bstatus = nullptr;
  uint32_t* bstatus_host = nullptr;   // pinned
  uint8_t* bplan_dev = nullptr;
  uint8_t* bplan_host = nullptr;      // pinned
  size_t bplan_cap = 0;
  uint32_t batch_tokens = 0, batch_hidden = 0;
};
Engine E;
bool g_open = false;
void release_engine();

size_t plan_capacity(uint32_t burst, uint32_t hidden) {
  // Pair or unit descriptors, then the group table, the decode token table
  // and unit indices, or the burst kernel's per-pair partial indices.
  return sizeof(PlanHeader) + (size_t)kMaxPlanPairs * sizeof(PairDesc) +
         (size_t)kMaxPlanPairs * kMaxBurst * sizeof(uint32_t) + kMaxBurst * sizeof(DecodeToken) + 256 +
         (size_t)burst * hidden * sizeof(float);
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// Pairs per down-phase group: about 48 KB of down weights per task.
// The group size is also capped so that phase B's LDS (the group's h for
// 8 tokens, the per-wave tables and the fp64 partial sums; the ldsB formula
// of build_plan) stays within kLdsLimit for any burst.
uint32_t group_pairs(uint8_t dn) {
  uint32_t per = dn == TQ4_KT ? 4608u : kCols * (uint32_t)row_bytes(dn, kNeurons);
  uint32_t cap = dn == TQ8_0 ? group_max<TQ8_0>() : dn == TQ4_KT ? group_max<TQ4_KT>() : group_max<TMXFP4>();
  constexpr size_t kWstride = 2 * 8 * kTabStride + kMaxBurst * 8 * kTabStride;
  constexpr size_t kFixed = kWaves * kWstride * sizeof(float) + kWaves * kCols * sizeof(double);
  constexpr uint32_t kLdsGroups = (uint32_t)((kLdsLimit - kFixed) / (kMaxBurst * kNeurons * sizeof(float)));
  static_assert(kLdsGroups >= 1, "one pair per group fits the LDS limit");
  if (cap > kLdsGroups) cap = kLdsGroups;
  uint32_t g = E.group_bytes / per;
  return g < 1 ? 1 : g > cap ? cap : g;
}

// The row-format kernel instantiation for a block's formats: (routed
// gate/up, down) and the shared expert's, or kNoCombo.
constexpr uint32_t kNoCombo = ~0u;
constexpr uint32_t kComboShared = 0x10;   // the request has shared-expert units
enum : uint32_t { COMBO_NATIVE = 0, COMBO_Q8 = 1, COMBO_MXFP4 = 2, COMBO_Q4_0 = 3 };
uint32_t rows_combo(const Layout& l) {
  if (l.gu == TQ4_K && l.dn == TMXFP4 && l.shared_gu == TQ8_0 && l.shared_dn == TQ8_0) return COMBO_NATIVE;
  if (l.gu == TQ8_0 && l.dn == TQ8_0 && l.shared_gu == TQ8_0 && l.shared_dn == TQ8_0) return COMBO_Q8;
  if (l.gu == TMXFP4 && l.dn == TMXFP4 && l.shared_gu == TQ8_0 && l.shared_dn == TQ8_0) return COMBO_MXFP4;
  if (l.gu == TQ4_0 && l.dn == TQ4_0 && l.shared_gu == TQ4_0 && l.shared_dn == TQ4_0) return COMBO_Q4_0;
  return kNoCombo;
}

int build_plan(const fr_hip_request* r, uint8_t* out, size_t cap, size_t* used, unsigned* grid) {
  if (!r || !out || !used || !grid || !r->expert || !r->gate || !r->x) return FR_HIP_INVALID;
  if (r->burst < 1 || r->burst > (unsigned)kMaxBurst || r->layer >= (unsigned)kLayers || r->mode > MODE_Q8_256)
    return FR_HIP_INVALID;
  const uint32_t T = r->burst, hidden = r->hidden;
  int nloaded = 0;
  for (int b = 0; b < kBlocks; ++b) {
    if (!E.block[b]) continue;
    if (E.lay[b].hidden != hidden) return FR_HIP_INVALID;
    ++nloaded;
  }
  if (!nloaded) return FR_HIP_STATE;
  for (int b = 0; b < kBlocks; ++b)
    if (E.block[b] && r->layer >= E.layers[b]) return FR_HIP_STATE;
  if (cap < plan_capacity(T, hidden)) return FR_HIP_INVALID;
  // Unique experts, token-major first appearance (backends/avx2.c:661-672).
  uint16_t ids[kMaxUnique];
  uint8_t masks[kMaxUnique] = {};
  float gates[kMaxUnique][kMaxBurst] = {};
  int nu = 0;
  for (uint32_t t = 0; t < T; ++t)
    for (int e = 0; e < 11; ++e) {
      float g = r->gate[t * 11 + e];
      if (e == 10 && g == 0.f) continue;
      uint16_t id = e == 10 ? (uint16_t)kShared : r->expert[t * 10 + e];
      if (e < 10 && id >= kShared) return FR_HIP_INVALID;   // routed ids < 512 (backends/ref.c:46)
      int s = 0;
      while (s < nu && ids[s] != id) ++s;
      if (s == nu) ids[nu++] = id;
      masks[s] |= (uint8_t)(1u << t);
      gates[s][t] = g;
    }
  // Route first, from the loaded blocks' layouts, so that a decode plan is
  // built alone (x copied once). F32, routed experts only (no shared gate),
  // every pair Q4_K with the transposed down: the decode kernel. Its work
  // list is rebuilt as (token, pair) units, token-major, each token's experts
  // in request order and blocks ascending (the single-token pair order), so
  // that a token's units and their summation order do not depend on the
  // rest of the burst. F32 and every pair one of the row-format pairs (shared
  // expert included): decode_rows_kernel, on the same work list. ref-q8
  // requests take the same two routes (decode_q8_kernel,
  // decode_rows_q8_kernel), the row formats only where gate/up dots in
  // integers (not MXFP4).
  PlanHeader* H = reinterpret_cast<PlanHeader*>(out);
  memset(H, 0, sizeof(*H));
  H->pairs_off = sizeof(PlanHeader);
  PairDesc* pairs = reinterpret_cast<PairDesc*>(out + sizeof(PlanHeader));
  uint64_t wbytes = 0;   // the request's weight bytes: each (expert, block) slice once
  for (int s2 = 0; s2 < nu; ++s2)
    for (int b = 0; b < kBlocks; ++b)
      if (E.block[b]) wbytes += ids[s2] == kShared ? E.lay[b].shared_slice : E.lay[b].slice;
  const bool fits = hidden <= (uint32_t)kMaxHidden && E.cus > 0;
  // The row-format kernel is instantiated per unit format: every loaded
  // block must have the first one's routed and shared formats.
  int first = 0;
  while (!E.block[first]) ++first;
  const uint32_t combo = rows_combo(E.lay[first]);
  // q8_256 is the AVX2 backend's arithmetic. With legacy Q4_0 blocks that
  // backend quantizes x per 64 into fr_q8_activation's codes
  // (backends/avx2.c:83-100 against src/q4.c:37-61, used when any block is
  // legacy, :630-633), so those requests run in the ref-q8 arithmetic.
  uint32_t mode = r->mode;
  if (mode == MODE_Q8_256) {
    bool legacy = true;
    for (int b = 0; b < kBlocks; ++b) legacy = legacy && (!E.block[b] || E.lay[b].gu == TQ4_0);
    if (legacy) mode = MODE_Q8;
  }
  const bool f32q8 = (mode == MODE_F32 || mode == MODE_Q8 || mode == MODE_Q8_256) && fits;
  bool q4kt = f32q8 && mode != MODE_Q8_256, rows = f32q8;
  rows = rows && combo != kNoCombo;
  // ref-q8 row units need integer gate/up dots (decode_rows_q8_kernel);
  // q8_256 runs on the native and Q8_0 units, the formats its backend knows.
  if (mode == MODE_Q8) rows = rows && (combo == COMBO_NATIVE || combo == COMBO_Q8 || combo == COMBO_Q4_0);
  if (mode == MODE_Q8_256) rows = rows && (combo == COMBO_NATIVE || combo == COMBO_Q8);
  for (int b = 0; rows && b < kBlocks; ++b)
    rows = !E.block[b] || rows_combo(E.lay[b]) == combo;
  for (int b = 0; q4kt && b < kBlocks; ++b)
    q4kt = !E.block[b] || (E.lay[b].gu == TQ4_KM && E.lay[b].dn == TQ4_KT);
  for (int s2 = 0; q4kt && s2 < nu; ++s2) q4kt = ids[s2] != kShared;
  uint32_t nunits = 0;
  for (uint32_t t = 0; t < T; ++t) nunits += (10u + (r->gate[t * 11 + 10] != 0.f ? 1u : 0u)) * (uint32_t)nloaded;
  const bool decode = (q4kt || rows) && nunits <= (uint32_t)kMaxDecodeUnits;
  // F32 all-Q4_K units of a node with few owned blocks are split into
  // items of fewer row-blocks (decode_split_kernel); the split depends on
  // the owned blocks only, never on the burst. Bursts of two or more tokens
  // on the unsplit route whose tokens share experts run one workgroup turn
  // per unique pair (decode_burst_kernel): it pays from about two routed
  // tokens per unique expert on average (10 T >= 2 unique); below that the
  // per-(token, pair) units are faster (measured: 4 tokens on one expert
  // set 28.9 against 47.9 us, a 4-token Zipf(1.1) burst with 1.3 tokens
  // per expert 58 against 52 us).
  const uint32_t split = q4kt && mode == MODE_F32 ? (nloaded <= 5 ? 4u : nloaded <= 11 ? 2u : 1u) : 1u;
  const bool burst_k = q4kt && mode == MODE_F32 && T >= 2 && split == 1 && !E.no_burst &&
                       (E.force_burst || 10u * T >= 2u * (uint32_t)nu);
  uint32_t np = 0;
  if (decode && !E.no_decode && burst_k) {
    DecodeToken tok[kMaxBurst];
    for (uint32_t t = 0, first = 0; t < T; ++t) {
      tok[t].first = first;
      tok[t].count = 10u * (uint32_t)nloaded;
      first += tok[t].count;
    }
    // Unique pairs, experts in first-appearance order and blocks ascending;
    // each with its tokens' gates and, per token, the partial index of the
    // (token, pair) unit in the token-major numbering of decode_kernel.
    np = (uint32_t)nu * (uint32_t)nloaded;
    H->groups_off = H->pairs_off + np * sizeof(PairDesc);
    memcpy(out + H->groups_off, tok, T * sizeof(DecodeToken));
    uint32_t* bpart = reinterpret_cast<uint32_t*>(out + H->groups_off + T * sizeof(DecodeToken));
    uint32_t w = 0;
    for (int s2 = 0; s2 < nu; ++s2) {
      uint8_t place[kMaxBurst] = {};
      for (uint32_t t = 0; t < T; ++t) {
        if (!(masks[s2] >> t & 1u)) continue;
        int e = 0;
        while (r->expert[t * 10 + e] != ids[s2]) ++e;
        place[t] = (uint8_t)e;
      }
      int brank = 0;
      for (int b = 0; b < kBlocks; ++b) {
        if (!E.block[b]) continue;
        const Layout& l = E.lay[b];
        PairDesc& P = pairs[w];
        memset(&P, 0, sizeof(P));
        P.slice = (uint64_t)(uintptr_t)(E.block[b] + (uint64_t)r->layer * l.layer + (uint64_t)ids[s2] * l.slice);
        P.proj = (uint32_t)l.proj;
        P.gu = (uint8_t)l.gu;
        P.dn = (uint8_t)l.dn;
        P.tmask = masks[s2];
        for (uint32_t t = 0; t < T; ++t) {
          P.gate[t] = gates[s2][t];
          bpart[w * kMaxBurst + t] =
              masks[s2] >> t & 1u ? tok[t].first + (uint32_t)place[t] * (uint32_t)nloaded + (uint32_t)brank : 0u;
        }
        for (uint32_t t = T; t < (uint32_t)kMaxBurst; ++t) bpart[w * kMaxBurst + t] = 0u;
        ++w;
        ++brank;
      }
    }
    if (w != np) return FR_HIP_INVALID;
    H->hidden = hidden;
    H->burst = T;
    H->mode = mode;
    H->npairs = np;
    H->ngroups = T;
    H->x_off = (uint32_t)((H->groups_off + T * sizeof(DecodeToken) + np * kMaxBurst * sizeof(uint32_t) + 255) & ~255u);
    memcpy(out + H->x_off, r->x, (size_t)T * hidden * sizeof(float));
    H->total = H->x_off + T * hidden * (uint32_t)sizeof(float);
    const uint32_t cap = E.cus < (unsigned)kDecodeGridMax ? E.cus : (unsigned)kDecodeGridMax;
    H->kind = KIND_DECODE_BURST;
    H->pad = 0;
    H->tpw = (np + cap - 1) / cap;
    H->grid = (np + H->tpw - 1) / H->tpw;
  } else if (decode && !E.no_decode) {
    // Units are (token, pair). Their partials are numbered token-major in the
    // reference's order (token, routed expert in request order, ascending
    // block), which the reduction follows; the work list is pair-major, so
    // that the units of one pair are consecutive in one workgroup's chunk and
    // its bytes are read again while they are still cached.
    DecodeToken tok[kMaxBurst];
    for (uint32_t t = 0, first = 0; t < T; ++t) {
      tok[t].first = first;
      tok[t].count = (10u + (r->gate[t * 11 + 10] != 0.f ? 1u : 0u)) * (uint32_t)nloaded;
      first += tok[t].count;
    }
    uint32_t* upart = reinterpret_cast<uint32_t*>(out + H->pairs_off + nunits * sizeof(PairDesc) +
                                                  T * sizeof(DecodeToken));
    uint32_t w = 0;
    for (int s2 = 0; s2 < nu; ++s2) {
      const bool shared = ids[s2] == kShared;
      // The expert's place in each of its tokens' lists (the shared expert
      // follows the 10 routed), found once for all blocks.
      uint8_t place[kMaxBurst] = {};
      for (uint32_t t = 0; t < T; ++t) {
        if (!(masks[s2] >> t & 1u)) continue;
        int e = 10;
        if (!shared) {
          e = 0;
          while (r->expert[t * 10 + e] != ids[s2]) ++e;
        }
        place[t] = (uint8_t)e;
      }
      int brank = 0;
      for (int b = 0; b < kBlocks; ++b) {
        if (!E.block[b]) continue;
        const Layout& l = E.lay[b];
        const uint64_t slice = (uint64_t)(uintptr_t)(E.block[b] + (uint64_t)r->layer * l.layer +
                                                     (uint64_t)ids[s2] * l.slice);
        for (uint32_t t = 0; t < T; ++t) {
          if (!(masks[s2] >> t & 1u)) continue;
          const int e = place[t];
          PairDesc& U = pairs[w];
          U.slice = slice;
          U.proj = (uint32_t)(shared ? l.shared_proj : l.proj);
          U.gu = (uint8_t)(shared ? l.shared_gu : l.gu);
          U.dn = (uint8_t)(shared ? l.shared_dn : l.dn);
          U.tmask = (uint8_t)(1u << t);
          U.pad = (uint8_t)t;
          U.gate[0] = r->gate[t * 11 + e];
          for (int k = 1; k < kMaxBurst; ++k) U.gate[k] = 0.f;
          upart[w++] = tok[t].first + (uint32_t)e * (uint32_t)nloaded + (uint32_t)brank;
        }
        ++brank;
      }
    }
    if (w != nunits) return FR_HIP_INVALID;   // every token routes 10 distinct experts
    if (w > (uint32_t)kMaxDecodeUnits) return FR_HIP_INVALID;
    H->hidden = hidden;
    H->burst = T;
    H->mode = mode;
    H->npairs = nunits;
    H->ngroups = T;
    H->groups_off = H->pairs_off + nunits * sizeof(PairDesc);
    memcpy(out + H->groups_off, tok, T * sizeof(DecodeToken));
    H->x_off = (uint32_t)((H->groups_off + T * sizeof(DecodeToken) + nunits * sizeof(uint32_t) + 255) & ~255u);
    memcpy(out + H->x_off, r->x, (size_t)T * hidden * sizeof(float));
    H->total = H->x_off + T * hidden * (uint32_t)sizeof(float);
    // One workgroup per CU at most, each taking a contiguous chunk of
    // ceil(items / cap) items of the work list.
    const uint32_t cap = E.cus < (unsigned)kDecodeGridMax ? E.cus : (unsigned)kDecodeGridMax;
    H->kind = q4kt ? KIND_DECODE : KIND_DECODE_ROWS;
    bool with_shared = false;
    for (uint32_t t = 0; t < T; ++t) with_shared = with_shared || r->gate[t * 11 + 10] != 0.f;
    H->pad = q4kt ? 0u : combo | (with_shared ? kComboShared : 0u);
    if (split > 1) {
      H->kind = KIND_DECODE_SPLIT;
      H->pad = split;
      DecodeToken* table = reinterpret_cast<DecodeToken*>(out + H->groups_off);   // a token's items
      for (uint32_t t = 0; t < T; ++t) {
        table[t].first *= split;
        table[t].count *= split;
      }
    }
    const uint32_t items = nunits * split;
    const uint32_t ppw = (items + cap - 1) / cap;
    H->tpw = ppw;
    H->grid = (items + ppw - 1) / ppw;
    np = nunits;
  } else if (mode == MODE_Q8_256) {
    return FR_HIP_UNSUPPORTED;   // the layer kernel has no q8_256 arithmetic
  } else {
    // Pairs, partitioned by down format so each group is homogeneous.
    uint8_t classes[4] = {TQ4_KT, TMXFP4, TQ4_0, TQ8_0};
    GroupDesc groups[kMaxPairs];
    uint32_t ng = 0, gmax = 1;
    for (uint8_t cls : classes) {
      uint32_t start = np;
      for (int s = 0; s < nu; ++s)
        for (int b = 0; b < kBlocks; ++b) {
          if (!E.block[b]) continue;
          const Layout& l = E.lay[b];
          bool shared = ids[s] == kShared;
          uint8_t dn = (uint8_t)(shared ? l.shared_dn : l.dn);
          if (dn != cls) continue;
          PairDesc& P = pairs[np++];
          memset(&P, 0, sizeof(P));
          P.slice = (uint64_t)(uintptr_t)(E.block[b] + (uint64_t)r->layer * l.layer + (uint64_t)ids[s] * l.slice);
          P.proj = (uint32_t)(shared ? l.shared_proj : l.proj);
          P.gu = (uint8_t)(shared ? l.shared_gu : l.gu);
          P.dn = dn;
          P.tmask = masks[s];
          for (uint32_t t = 0; t < T; ++t) P.gate[t] = gates[s][t];
        }
      uint32_t gp = group_pairs(cls);
      for (uint32_t f = start; f < np; f += gp) {
        GroupDesc& G = groups[ng++];
        memset(&G, 0, sizeof(G));
        G.first = (uint16_t)f;
        G.count = (uint16_t)(np - f < gp ? np - f : gp);
        G.dn = cls;
        if (G.count > gmax) gmax = G.count;
      }
    }
    const uint32_t nn = kTaskNeurons;
    H->hidden = hidden;
    H->burst = T;
    H->mode = mode;
    H->npairs = np;
    H->ngroups = ng;
    H->nranges = hidden / kCols;
    H->nn = nn;
    H->ntA = np * (kNeurons / nn);
    H->ntB = ng * H->nranges;
    // Phase A stages activations in tiles of 1 (single token) or 4 tokens.
    const uint32_t tchunk = T == 1 ? 1 : (T < 4 ? T : 4);
    H->tchunk = tchunk;
    H->gmax = gmax;
    H->groups_off = H->pairs_off + np * sizeof(PairDesc);
    memcpy(out + H->groups_off, groups, ng * sizeof(GroupDesc));
    H->x_off = (uint32_t)((H->groups_off + ng * sizeof(GroupDesc) + 255) & ~255u);
    memcpy(out + H->x_off, r->x, (size_t)T * hidden * sizeof(float));
    H->total = H->x_off + T * hidden * (uint32_t)sizeof(float);
    size_t ldsA = T == 1 ? 0 : (size_t)tchunk * hidden * sizeof(float);
    size_t wstride = 2 * 8 * kTabStride + T * 8 * kTabStride;
    size_t ldsB = (size_t)gmax * T * kNeurons * sizeof(float) + kWaves * wstride * sizeof(float) +
                  kWaves * kCols * sizeof(double);
    H->lds = (uint32_t)(ldsA > ldsB ? ldsA : ldsB);
    if (H->lds > (uint32_t)kLdsLimit) return FR_HIP_UNSUPPORTED;
    H->kind = KIND_LAYER;
    H->tpw = 0;
    H->grid = H->ntA + H->ntB;
  }
  *used = H->total;
  *grid = H->grid;
  E.sample.unique_experts = (unsigned)nu;
  E.sample.pairs = np;
  E.sample.grid = *grid;
  E.sample.blocks = (unsigned)nloaded;
  E.sample.weight_bytes = wbytes;
  return FR_HIP_OK;
}

// A decode plan's token table lies within the plan (launch_decode copies it
// from the host plan into the kernel arguments).
bool decode_table_ok(const PlanHeader& H) {
  return H.groups_off >= sizeof(PlanHeader) && (uint64_t)H.groups_off + H.burst * sizeof(DecodeToken) <= H.total;
}

// decode_kernel or the decode_rows_kernel instantiation of the plan's unit
// formats, then decode_reduce, on `stream`; `mid`, if set, is recorded
// between them. Returns false if an event could not be recorded.
bool launch_decode(const uint8_t* dev_plan, const PlanHeader& H, unsigned grid, const Scratch& S0, hipStream_t stream,
                   hipEvent_t mid) {
  const dim3 g(grid), b(kDecodeThreads);
  // The header's fields and the token table (at groups_off of the host plan
  // H heads; every caller checks that it lies within the plan).
  Scratch S = S0;
  S.A.hidden = H.hidden;
  S.A.burst = H.burst;
  S.A.npairs = H.npairs;
  S.A.tpw = H.tpw;
  S.A.pairs_off = H.pairs_off;
  S.A.groups_off = H.groups_off;
  S.A.x_off = H.x_off;
  S.A.pad = 0;
  memset(S.A.tok, 0, sizeof(S.A.tok));
  memcpy(S.A.tok, reinterpret_cast<const uint8_t*>(&H) + H.groups_off, H.burst * sizeof(DecodeToken));
  // decode_q8_kernel or decode_rows_q8_kernel: double partials.
  const bool q8 = H.mode == MODE_Q8 || H.mode == MODE_Q8_256;
  if (H.kind == KIND_DECODE_BURST) hipLaunchKernelGGL(decode_burst_kernel, g, b, 0, stream, dev_plan, S);
  else if (H.kind == KIND_DECODE_SPLIT && H.pad == 4) hipLaunchKernelGGL(decode_split_kernel<1>, g, b, 0, stream, dev_plan, S);
  else if (H.kind == KIND_DECODE_SPLIT) hipLaunchKernelGGL(decode_split_kernel<2>, g, b, 0, stream, dev_plan, S);
  else if (H.kind == KIND_DECODE && q8) hipLaunchKernelGGL(decode_q8_kernel, g, b, 0, stream, dev_plan, S);
  else if (H.kind == KIND_DECODE) hipLaunchKernelGGL(decode_kernel, g, b, 0, stream, dev_plan, S);
  else if (H.mode == MODE_Q8_256) switch (H.pad) {   // native or Q8_0 units only (build_plan, launch)
    case COMBO_NATIVE:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ4_K, TMXFP4, TQ4_K, TMXFP4, true>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_NATIVE | kComboShared:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ4_K, TMXFP4, TQ8_0, TQ8_0, true>), g, b, 0, stream, dev_plan, S);
      break;
    default:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ8_0, TQ8_0, TQ8_0, TQ8_0, true>), g, b, 0, stream, dev_plan, S);
      break;
  }
  else if (q8) switch (H.pad) {   // the integer gate/up formats only (build_plan)
    case COMBO_NATIVE:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ4_K, TMXFP4, TQ4_K, TMXFP4>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_NATIVE | kComboShared:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ4_K, TMXFP4, TQ8_0, TQ8_0>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_Q8:
    case COMBO_Q8 | kComboShared:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ8_0, TQ8_0, TQ8_0, TQ8_0>), g, b, 0, stream, dev_plan, S);
      break;
    default:
      hipLaunchKernelGGL((decode_rows_q8_kernel<TQ4_0, TQ4_0, TQ4_0, TQ4_0>), g, b, 0, stream, dev_plan, S);
      break;
  }
  else switch (H.pad) {   // (routed formats, shared formats) of the units the request has
    case COMBO_NATIVE:
      hipLaunchKernelGGL((decode_rows_kernel<TQ4_K, TMXFP4, TQ4_K, TMXFP4>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_NATIVE | kComboShared:
      hipLaunchKernelGGL((decode_rows_kernel<TQ4_K, TMXFP4, TQ8_0, TQ8_0>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_Q8:
    case COMBO_Q8 | kComboShared:
      hipLaunchKernelGGL((decode_rows_kernel<TQ8_0, TQ8_0, TQ8_0, TQ8_0>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_MXFP4:
      hipLaunchKernelGGL((decode_rows_kernel<TMXFP4, TMXFP4, TMXFP4, TMXFP4>), g, b, 0, stream, dev_plan, S);
      break;
    case COMBO_MXFP4 | kComboShared:
      hipLaunchKernelGGL((decode_rows_kernel<TMXFP4, TMXFP4, TQ8_0, TQ8_0>), g, b, 0, stream, dev_plan, S);
      break;
    default:
      hipLaunchKernelGGL((decode_rows_kernel<TQ4_0, TQ4_0, TQ4_0, TQ4_0>), g, b, 0, stream, dev_plan, S);
      break;
  }
  if (mid && hipEventRecord(mid, stream) != hipSuccess) return false;
  if (q8)
    hipLaunchKernelGGL(decode_reduce<true>, dim3(kMaxHidden / kReducePositions, H.burst), dim3(kReduceThreads), 0,
                       stream, dev_plan, S);
  else
    hipLaunchKernelGGL(decode_reduce<false>, dim3(kMaxHidden / kReducePositions, H.burst), dim3(kReduceThreads), 0,
                       stream, dev_plan, S);
  return true;
}

// Copies a plan from mapped pinned host memory into device memory, one
// 16-byte word per lane with every load in flight at once: one PCIe round
// trip, where a DMA copy first waits for its engine and then for the kernels'
// queue (about 4 us more per run, measured).
__global__ __launch_bounds__(64) void stage_plan(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                 unsigned words) {
  const unsigned i = blockIdx.x * 64 + threadIdx.x;
  if (i < words) dst[i] = src[i];
}

// `host`: a decode plan's y and status words go to the engine's mapped host
// buffers (fr_hip_run), and the engine's output parity is left as it is.
int launch(const uint8_t* dev_plan, const PlanHeader& H, unsigned grid, hipStream_t stream, bool host = false) {
  if ((size_t)H.ngroups * H.burst * H.hidden * sizeof(double) > E.partial_bytes) return FR_HIP_UNSUPPORTED;
  const bool decode = H.kind == KIND_DECODE || H.kind == KIND_DECODE_ROWS || H.kind == KIND_DECODE_SPLIT ||
                      H.kind == KIND_DECODE_BURST;
  const unsigned items = H.kind == KIND_DECODE_SPLIT ? H.npairs * H.pad : H.npairs;
  if (H.kind == KIND_DECODE_SPLIT && H.pad != 2 && H.pad != 4) return FR_HIP_INVALID;
  // A burst plan's partials: 10 routed experts x the owned blocks per token.
  if (H.kind == KIND_DECODE_BURST && (H.mode != MODE_F32 || H.burst < 2 || H.npairs > (unsigned)kMaxPairs ||
                                      H.burst * 10u * (unsigned)kBlocks > (unsigned)kMaxDecodeItems))
    return FR_HIP_INVALID;
  if (decode && (grid > (unsigned)kDecodeGridMax || grid > items || items > (unsigned)kMaxDecodeItems ||
                 H.ngroups != H.burst))
    return FR_HIP_INVALID;
  if (H.kind == KIND_DECODE_ROWS && (H.pad & ~kComboShared) > COMBO_Q4_0) return FR_HIP_INVALID;
  if (H.mode > MODE_Q8_256) return FR_HIP_INVALID;
  if (H.mode == MODE_Q8_256 && (H.kind != KIND_DECODE_ROWS || ((H.pad & ~kComboShared) != COMBO_NATIVE &&
                                                               (H.pad & ~kComboShared) != COMBO_Q8)))
    return FR_HIP_INVALID;
  Scratch S;
  S.done = E.done;
  S.fin = E.fin;
  S.hbuf = E.hbuf;
  S.partial = E.partial;
  S.out = E.out;
  S.wgpart = E.wgpart;
  S.bar = E.bar;
  S.out_words = E.out_words;
  S.parity = E.parity;
  S.ustride = kMaxDecodeItems;
  S.ystat = nullptr;
  S.yout = nullptr;
  S.dstat = nullptr;
  S.hstat = nullptr;
  host = host && decode;
  if (host) {
    S.hstat = E.hstat_dev;
    S.yout = E.hy_dev;
    S.dstat = E.hdstat;
  }
  const dim3 g(grid), blk(kThreads);
  const bool one = H.burst == 1;
  hipEvent_t* te = E.timing && E.timed < E.timed_cap ? E.tev + 3 * E.timed++ : nullptr;
  if (te && hipEventRecord(te[0], stream) != hipSuccess) return FR_HIP_IO;
  if (decode) {
    if (!launch_decode(dev_plan, H, grid, S, stream, te ? te[1] : nullptr)) return FR_HIP_IO;
  } else switch (H.mode) {
    case MODE_F32:
      if (one) hipLaunchKernelGGL((layer_kernel<MODE_F32, 1>), g, blk, H.lds, stream, dev_plan, S);
      else hipLaunchKernelGGL((layer_kernel<MODE_F32, 8>), g, blk, H.lds, stream, dev_plan, S);
      break;
    case MODE_F64:
      if (one) hipLaunchKernelGGL((layer_kernel<MODE_F64, 1>), g, blk, H.lds, stream, dev_plan, S);
      else hipLaunchKernelGGL((layer_kernel<MODE_F64, 8>), g, blk, H.lds, stream, dev_plan, S);
      break;
    default:
      if (one) hipLaunchKernelGGL((layer_kernel<MODE_Q8, 1>), g, blk, H.lds, stream, dev_plan, S);
      else hipLaunchKernelGGL((layer_kernel<MODE_Q8, 8>), g, blk, H.lds, stream, dev_plan, S);
      break;
  }
  if (te) {
    if (!decode && hipEventRecord(te[1], stream) != hipSuccess) return FR_HIP_IO;
    if (hipEventRecord(te[2], stream) != hipSuccess) return FR_HIP_IO;
  }
  if (hipGetLastError() != hipSuccess) return FR_HIP_IO;
  if (!host) {
    E.last_parity = E.parity;
    E.parity ^= 1u;
  }
  return FR_HIP_OK;
}

#define CK(x) do { if ((x) != hipSuccess) return FR_HIP_IO; } while (0)

// Copy the last launch's status word and fp32 outputs to pinned host memory,
// stream-ordered. The kernel already applied the reference's narrowing rule
// (backends/ref.c:37-40, 95): a non-finite or beyond-FLT_MAX sum sets a
// status bit and the caller returns FR_NUMERIC.
int fetch_output(hipStream_t s, size_t count, float* y, unsigned* status_out) {
  const uint32_t* src = E.out + (size_t)E.last_parity * E.out_words;
  CK(hipMemcpyAsync(E.out_host, src, (4 + count) * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  CK(hipStreamSynchronize(s));
  if (status_out) *status_out = E.out_host[0];
  if (y && !E.out_host[0]) memcpy(y, E.out_host + 4, count * sizeof(float));
  return FR_HIP_OK;
}

// ------------------------------------------------------------ prefill plan

size_t batch_capacity(uint32_t tokens, uint32_t hidden) {
  const size_t slots = (size_t)tokens * 11;
  return sizeof(BatchHeader) + slots * (sizeof(BatchTile) + sizeof(BatchSlot) + sizeof(uint32_t)) + 4 * 256 +
         (size_t)tokens * hidden * sizeof(float);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Tokens grouped by routed expert (ascending id), each expert's tokens in
// ascending order, cut into tiles of at most 16, then the tokens with the
// shared expert (slots 10T..) in tiles of their own; tokslot[t][e] is the
// slot of token t's e-th expert (e = 10: the shared expert, or kNoSlot), the
// order in which its partials are summed (backends/ref.c:61-97). Every
// loaded block has one format: Q4_K-T units (routed on prefill_gate_up /
// prefill_down) or native units (Q4_K rows, MXFP4 down: the row-format
// prefill kernels); the shared expert is Q8_0 in both.
int build_batch(const fr_hip_batch* r, uint8_t* out, size_t cap, size_t* used) {
  if (!r || !out || !used || !r->expert || !r->gate || !r->x) return FR_HIP_INVALID;
  if (!r->tokens || r->tokens > (unsigned)kMaxBatchTokens || r->layer >= (unsigned)kLayers || r->mode > MODE_Q8_256)
    return FR_HIP_INVALID;
  if (r->mode != MODE_F32) return FR_HIP_UNSUPPORTED;
  const uint32_t T = r->tokens, hidden = r->hidden;
  if (cap < batch_capacity(T, hidden)) return FR_HIP_INVALID;
  BatchHeader* H = reinterpret_cast<BatchHeader*>(out);
  memset(H, 0, sizeof(*H));
  const Layout* l0 = nullptr;
  for (int b = 0; b < kBlocks; ++b) {
    if (!E.block[b]) continue;
    const Layout& l = E.lay[b];
    if (l.hidden != hidden) return FR_HIP_INVALID;
    const bool kt = l.gu == TQ4_KM && l.dn == TQ4_KT, nat = l.gu == TQ4_K && l.dn == TMXFP4;
    if (!(kt || nat) || l.shared_gu != TQ8_0 || l.shared_dn != TQ8_0) return FR_HIP_UNSUPPORTED;
    if (l0 && (l.gu != l0->gu || l.dn != l0->dn)) return FR_HIP_UNSUPPORTED;
    if (r->layer >= E.layers[b]) return FR_HIP_STATE;
    H->base[H->nblk++] = (uint64_t)(uintptr_t)(E.block[b] + (uint64_t)r->layer * l.layer);
    l0 = &l;
  }
  if (!l0) return FR_HIP_STATE;
  std::vector<uint32_t> count(kRouted, 0), first(kRouted, 0), fill(kRouted, 0);
  uint32_t nshared = 0;
  for (uint32_t t = 0; t < T; ++t) {
    nshared += r->gate[t * 11 + 10] != 0.f ? 1u : 0u;
    for (int e = 0; e < 10; ++e) {
      const uint16_t id = r->expert[t * 10 + e];
      if (id >= kRouted) return FR_HIP_INVALID;
      for (int f = 0; f < e; ++f)
        if (r->expert[t * 10 + f] == id) return FR_HIP_INVALID;
      ++count[id];
    }
  }
  uint32_t nslots = 0, ntiles = 0, experts = 0;
  for (int id = 0; id < kRouted; ++id) {
    first[id] = nslots;
    nslots += count[id];
    ntiles += (count[id] + kTileTokens - 1) / kTileTokens;
    experts += count[id] ? 1u : 0u;
  }
  const uint32_t shtiles = (nshared + kTileTokens - 1) / kTileTokens;
  H->hidden = hidden;
  H->tokens = T;
  H->nslots = nslots + nshared;
  H->ntiles = ntiles;
  H->nshared = nshared;
  H->shtiles = shtiles;
  H->gu = l0->gu;
  H->dn = l0->dn;
  H->layer = r->layer;
  H->experts = experts;
  H->slice_bytes = l0->slice;
  H->proj = l0->proj;
  H->shared_proj = l0->shared_proj;
  H->tiles_off = (uint32_t)align256(sizeof(BatchHeader));
  H->slots_off = (uint32_t)align256(H->tiles_off + (size_t)(ntiles + shtiles) * sizeof(BatchTile));
  H->tokslot_off = (uint32_t)align256(H->slots_off + (size_t)H->nslots * sizeof(BatchSlot));
  H->x_off = (uint32_t)align256(H->tokslot_off + (size_t)T * 11 * sizeof(uint32_t));
  H->total = H->x_off + T * hidden * (uint32_t)sizeof(float);
  BatchTile* tiles = reinterpret_cast<BatchTile*>(out + H->tiles_off);
  BatchSlot* slots = reinterpret_cast<BatchSlot*>(out + H->slots_off);
  uint32_t* tokslot = reinterpret_cast<uint32_t*>(out + H->tokslot_off);
  for (uint32_t t = 0; t < T; ++t)
    for (int e = 0; e < 10; ++e) {
      const uint16_t id = r->expert[t * 10 + e];
      const uint32_t s = first[id] + fill[id]++;
      slots[s].token = t;
      slots[s].gate = r->gate[t * 11 + e];
      tokslot[t * 11 + e] = s;
    }
  for (uint32_t t = 0, k = 0; t < T; ++t) {
    tokslot[t * 11 + 10] = kNoSlot;
    if (r->gate[t * 11 + 10] == 0.f) continue;
    slots[nslots + k].token = t;
    slots[nslots + k].gate = r->gate[t * 11 + 10];
    tokslot[t * 11 + 10] = nslots + k++;
  }
  uint32_t k = 0;
  for (int id = 0; id < kRouted; ++id)
    for (uint32_t f = 0; f < count[id]; f += kTileTokens) {
      BatchTile& B = tiles[k++];
      B.expert = (uint32_t)id;
      B.ntok = count[id] - f < (uint32_t)kTileTokens ? count[id] - f : (uint32_t)kTileTokens;
      B.slot0 = first[id] + f;
      B.pad = 0;
    }
  for (uint32_t f = 0; f < nshared; f += kTileTokens) {
    BatchTile& B = tiles[k++];
    B.expert = (uint32_t)kShared;
    B.ntok = nshared - f < (uint32_t)kTileTokens ? nshared - f : (uint32_t)kTileTokens;
    B.slot0 = nslots + f;
    B.pad = 0;
  }
  memcpy(out + H->x_off, r->x, (size_t)T * hidden * sizeof(float));
  *used = H->total;
  E.sample.unique_experts = experts;
  E.sample.pairs = ntiles * H->nblk;
  E.sample.grid = ntiles;
  E.sample.blocks = H->nblk;
  E.sample.weight_bytes = (uint64_t)experts * H->nblk * l0->slice + (nshared ? H->nblk * l0->shared_slice : 0);
  return FR_HIP_OK;
}

// Scratch of the prefill kernels, grown on demand (never inside a timed
// region once warm: the sizes depend only on the token count).
int batch_scratch(const BatchHeader& H) {
  const size_t hb = (size_t)H.nslots * H.nblk * kNeurons * sizeof(float);
  const size_t pb = (size_t)H.nslots * H.hidden * sizeof(float);
  const size_t yb = (size_t)H.tokens * H.hidden * sizeof(float);
  if (hb > E.bh_bytes) {
    (void)hipFree(E.bh);
    E.bh = nullptr;
    E.bh_bytes = 0;
    CK(hipMalloc(&E.bh, hb));
    E.bh_bytes = hb;
    ++E.sample.hot_allocations;
  }
  if (pb > E.bpart_bytes) {
    (void)hipFree(E.bpart);
    E.bpart = nullptr;
    E.bpart_bytes = 0;
    CK(hipMalloc(&E.bpart, pb));
    E.bpart_bytes = pb;
    ++E.sample.hot_allocations;
  }
  const size_t db = (size_t)H.tokens * ((H.hidden / 256) * (1024 + 8 * sizeof(float)) + sizeof(float));
  if (db > E.bdig_bytes) {
    (void)hipFree(E.bdig);
    E.bdig = nullptr;
    E.bdig_bytes = 0;
    CK(hipMalloc(&E.bdig, db));
    E.bdig_bytes = db;
    ++E.sample.hot_allocations;
  }
  if (yb > E.by_bytes) {
    (void)hipFree(E.by);
    E.by = nullptr;
    E.by_bytes = 0;
    CK(hipMalloc(&E.by, yb));
    E.by_bytes = yb;
    ++E.sample.hot_allocations;
  }
  return FR_HIP_OK;
}

int batch_launch(const uint8_t* dev_plan, const BatchHeader& H, hipStream_t stream) {
  if (!H.tokens || H.tokens > (unsigned)kMaxBatchTokens || !H.ntiles || !H.nblk || H.nblk > (unsigned)kBlocks ||
      !H.hidden || H.hidden % 256 || H.hidden > (unsigned)kMaxHidden || H.nshared > H.tokens ||
      H.nslots != 10 * H.tokens + H.nshared || H.shtiles != (H.nshared + kTileTokens - 1) / kTileTokens)
    return FR_HIP_INVALID;
  const bool kt = H.gu == TQ4_KM && H.dn == TQ4_KT, nat = H.gu == TQ4_K && H.dn == TMXFP4;
  if (!kt && !nat) return FR_HIP_INVALID;
  int rc = batch_scratch(H);
  if (rc) return rc;
  BatchScratch S;
  S.h = E.bh;
  S.part = E.bpart;
  S.y = E.by;
  const size_t nd = (size_t)H.tokens * (H.hidden / 256);
  S.xh = reinterpret_cast<uint16_t*>(E.bdig);
  S.dsum = reinterpret_cast<float*>(E.bdig + nd * 1024);
  S.dscale = S.dsum + nd * 8;
  S.status = E.bstatus;
  hipEvent_t* te = E.timing && E.timed < E.timed_cap ? E.tev + 3 * E.timed++ : nullptr;
  CK(hipMemsetAsync(E.bstatus, 0, sizeof(uint32_t), stream));
  if (te) CK(hipEventRecord(te[0], stream));
  const unsigned ncol = (H.hidden + kDownCols - 1) / kDownCols;
  hipLaunchKernelGGL(prefill_split, dim3(H.tokens), dim3(1024), 0, stream, dev_plan, S);
  if (kt) hipLaunchKernelGGL(prefill_gate_up, dim3(H.ntiles * H.nblk), dim3(kBatchThreads), 0, stream, dev_plan, S);
  else
    hipLaunchKernelGGL(prefill_gate_up_rows<TQ4_K>, dim3(H.ntiles * H.nblk), dim3(kBatchThreads), 0, stream, dev_plan,
                       S, 0u);
  if (H.shtiles)
    hipLaunchKernelGGL(prefill_gate_up_rows<TQ8_0>, dim3(H.shtiles * H.nblk), dim3(kBatchThreads), 0, stream,
                       dev_plan, S, H.ntiles);
  const unsigned ncol_mx = (H.hidden + down_rows_cols<TMXFP4>() - 1) / down_rows_cols<TMXFP4>();
  const unsigned ncol_q8 = (H.hidden + down_rows_cols<TQ8_0>() - 1) / down_rows_cols<TQ8_0>();
  if (kt)
    hipLaunchKernelGGL(prefill_down, dim3(H.ntiles, (H.hidden + kDownWgCols - 1) / kDownWgCols), dim3(kDownThreads), 0,
                       stream, dev_plan, S);
  else
    hipLaunchKernelGGL(prefill_down_rows<TMXFP4>, dim3(H.ntiles, ncol_mx), dim3(kBatchThreads), 0, stream, dev_plan,
                       S, 0u);
  if (H.shtiles)
    hipLaunchKernelGGL(prefill_down_rows<TQ8_0>, dim3(H.shtiles, ncol_q8), dim3(kBatchThreads), 0, stream, dev_plan,
                       S, H.ntiles);
  if (te) CK(hipEventRecord(te[1], stream));
  hipLaunchKernelGGL(prefill_reduce, dim3(H.tokens, ncol), dim3(256), 0, stream, dev_plan, S);
  if (te) CK(hipEventRecord(te[2], stream));
  if (hipGetLastError() != hipSuccess) return FR_HIP_IO;
  E.batch_tokens = H.tokens;
  E.batch_hidden = H.hidden;
  return FR_HIP_OK;
}

int batch_output(hipStream_t s, float* y, size_t count, unsigned* status_out) {
  if (count > (size_t)E.batch_tokens * E.batch_hidden) return FR_HIP_INVALID;
  uint32_t status = 0;
  CK(hipMemcpyAsync(E.bstatus_host, E.bstatus, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  CK(hipStreamSynchronize(s));
  status = *E.bstatus_host;
  if (status_out) *status_out = status;
  if (y && count && !status) CK(hipMemcpy(y, E.by, count * sizeof(float), hipMemcpyDeviceToHost));
  return FR_HIP_OK;
}

}  // namespace

extern "C" {

int fr_hip_probe(int device, char* arch, size_t cap) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return FR_HIP_UNSUPPORTED;
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, device) != hipSuccess) return FR_HIP_UNSUPPORTED;
  if (arch && cap) snprintf(arch, cap, "%s", p.gcnArchName);
  return strncmp(p.gcnArchName, "gfx950", 6) ? FR_HIP_UNSUPPORTED : FR_HIP_OK;
}

uint64_t fr_hip_unit_bytes(unsigned hidden, unsigned format) {
  Layout l;
  return layout_of(hidden, format, l) ? l.block : 0;
}

int fr_hip_capacity(int device, unsigned hidden, unsigned format, uint64_t reserve, uint64_t* free_bytes,
                    unsigned* blocks) {
  if (!free_bytes || !blocks) return FR_HIP_INVALID;
  Layout l;
  if (!layout_of(hidden, format, l)) return FR_HIP_INVALID;
  int rc = fr_hip_probe(device, nullptr, 0);
  if (rc) return rc;
  int previous = 0;
  CK(hipGetDevice(&previous));
  CK(hipSetDevice(device));
  size_t avail = 0, total = 0;
  const hipError_t e = hipMemGetInfo(&avail, &total);
  CK(hipSetDevice(previous));
  if (e != hipSuccess) return FR_HIP_IO;
  // Units this engine already holds on the device count as available: the
  // figure is the device's capacity for units, not what is left of it.
  uint64_t held = 0;
  if (g_open && E.device == device)
    for (int b = 0; b < kBlocks; ++b)
      if (E.block[b]) held += E.lay[b].block;
  const uint64_t usable = (uint64_t)avail + held;
  const uint64_t n = usable > reserve ? (usable - reserve) / l.block : 0;
  *free_bytes = (uint64_t)avail;
  *blocks = n > (uint64_t)kBlocks ? (unsigned)kBlocks : (unsigned)n;
  return FR_HIP_OK;
}

static int open_engine(int device);

int fr_hip_open(int device) {
  if (g_open) return E.device == device ? FR_HIP_OK : FR_HIP_STATE;
  int rc = fr_hip_probe(device, nullptr, 0);
  if (rc) return rc;
  CK(hipSetDevice(device));
  E = Engine();
  E.device = device;
  rc = open_engine(device);
  if (rc) release_engine();   // nothing of a failed open stays allocated
  return rc;
}

// fr_hip_open's allocations; on failure the caller releases what exists.
static int open_engine(int device) {
  int cus = 0;
  CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  E.cus = cus > 0 ? (unsigned)cus : 1u;
  CK(hipStreamCreateWithFlags(&E.stream, hipStreamNonBlocking));
  CK(hipMalloc(&E.done, 2 * kMaxPairs * sizeof(uint32_t)));
  CK(hipMalloc(&E.fin, 2 * kMaxRanges * sizeof(uint32_t)));
  CK(hipMalloc(&E.hbuf, (size_t)kMaxPairs * kMaxBurst * kNeurons * sizeof(float)));
  // Group partials: at most one group per pair, bounded by the group byte cap.
  E.partial_bytes = (size_t)kMaxPairs * kMaxBurst * kMaxHidden * sizeof(double) / 4;
  CK(hipMalloc(&E.partial, E.partial_bytes));
  E.out_words = 4 + kMaxBurst * kMaxHidden;
  CK(hipMalloc(&E.out, 2 * (size_t)E.out_words * sizeof(uint32_t)));
  CK(hipMalloc(&E.wgpart, (size_t)kMaxDecodeItems * kMaxHidden * sizeof(double)));   // ref-q8 partials are doubles
  CK(hipMalloc(&E.bar, 2 * sizeof(uint32_t)));
  CK(hipMemset(E.bar, 0, 2 * sizeof(uint32_t)));
  // The static scratch array's address on this device (the name is a host
  // stand-in); it starts zeroed, as the error word must.
  CK(hipGetSymbolAddress(reinterpret_cast<void**>(&E.static_scratch), HIP_SYMBOL(scratch)));
  CK(hipHostMalloc(reinterpret_cast<void**>(&E.hy_host), (size_t)kMaxBurst * kMaxHidden * sizeof(float),
                   hipHostMallocMapped));
  CK(hipHostGetDevicePointer(reinterpret_cast<void**>(&E.hy_dev), E.hy_host, 0));
  CK(hipHostMalloc(reinterpret_cast<void**>(&E.hstat_host),
                   (size_t)kMaxBurst * (kMaxHidden / kReducePositions) * sizeof(uint32_t), hipHostMallocMapped));
  CK(hipHostGetDevicePointer(reinterpret_cast<void**>(&E.hstat_dev), E.hstat_host, 0));
  CK(hipMalloc(&E.hdstat, sizeof(uint32_t)));
  CK(hipMemset(E.hdstat, 0, sizeof(uint32_t)));
  E.group_bytes = (uint32_t)env_int("FRONK_HIP_GROUP_BYTES", 49152);
  E.no_decode = env_int("FRONK_HIP_NO_DECODE", 0) != 0;
  E.no_burst = false;
  E.force_burst = false;
  CK(hipMemset(E.done, 0, 2 * kMaxPairs * sizeof(uint32_t)));
  CK(hipMemset(E.fin, 0, 2 * kMaxRanges * sizeof(uint32_t)));
  CK(hipMemset(E.out, 0, 2 * (size_t)E.out_words * sizeof(uint32_t)));
  E.plan_cap = plan_capacity(kMaxBurst, kMaxHidden);
  // Rounded to whole 16-byte words for stage_plan.
  CK(hipMalloc(&E.plan_dev, (E.plan_cap + 15) & ~size_t(15)));
  CK(hipHostMalloc(reinterpret_cast<void**>(&E.plan_host), (E.plan_cap + 15) & ~size_t(15), hipHostMallocMapped));
  {
    void* mapped = nullptr;
    CK(hipHostGetDevicePointer(&mapped, E.plan_host, 0));
    E.plan_mapped = static_cast<const uint4*>(mapped);
  }
  CK(hipHostMalloc(reinterpret_cast<void**>(&E.out_host), (size_t)E.out_words * sizeof(uint32_t), hipHostMallocDefault));
  CK(hipMalloc(&E.bstatus, sizeof(uint32_t)));
  CK(hipMemset(E.bstatus, 0, sizeof(uint32_t)));
  CK(hipHostMalloc(reinterpret_cast<void**>(&E.bstatus_host), sizeof(uint32_t), hipHostMallocDefault));
  CK(hipEventCreate(&E.ev0));
  CK(hipEventCreate(&E.ev1));
  CK(hipEventCreate(&E.pev0));
  CK(hipEventCreate(&E.pev1));
  CK(hipDeviceSynchronize());
  g_open = true;
  return FR_HIP_OK;
}

int fr_hip_close(void) {
  if (!g_open) return FR_HIP_OK;
  for (int b = 0; b < kBlocks; ++b)
    if (E.block[b]) return FR_HIP_STATE;
  release_engine();
  return FR_HIP_OK;
}

}  // extern "C"

namespace {
// Frees whatever the engine holds (null handles are skipped) and resets it:
// fr_hip_close, and fr_hip_open when one of its steps fails.
void release_engine() {
  (void)hipSetDevice(E.device);
  if (E.stream) (void)hipStreamSynchronize(E.stream);
  (void)hipFree(E.done);
  (void)hipFree(E.fin);
  (void)hipFree(E.hbuf);
  (void)hipFree(E.partial);
  (void)hipFree(E.out);
  (void)hipFree(E.wgpart);
  (void)hipFree(E.bar);
  (void)hipFree(E.plan_dev);
  (void)hipFree(E.staging);
  (void)hipFree(E.bh);
  (void)hipFree(E.bpart);
  (void)hipFree(E.by);
  (void)hipFree(E.bdig);
  (void)hipFree(E.bstatus);
  (void)hipFree(E.bplan_dev);
  (void)hipHostFree(E.bplan_host);
  (void)hipHostFree(E.bstatus_host);
  (void)hipHostFree(E.plan_host);
  (void)hipHostFree(E.out_host);
  (void)hipHostFree(E.hy_host);
  (void)hipHostFree(E.hstat_host);
  (void)hipFree(E.hdstat);
  if (E.ev0) (void)hipEventDestroy(E.ev0);
  if (E.ev1) (void)hipEventDestroy(E.ev1);
  if (E.pev0) (void)hipEventDestroy(E.pev0);
  if (E.pev1) (void)hipEventDestroy(E.pev1);
  for (unsigned i = 0; i < 3 * E.timed_cap; ++i) (void)hipEventDestroy(E.tev[i]);
  free(E.tev);
  if (E.stream) (void)hipStreamDestroy(E.stream);
  E = Engine();
  g_open = false;
}
}  // namespace

extern "C" {

static int ensure_staging(size_t bytes) {
  if (E.staging_bytes >= bytes) return FR_HIP_OK;
  if (E.staging) (void)hipFree(E.staging);
  E.staging = nullptr;
  E.staging_bytes = 0;
  CK(hipMalloc(&E.staging, bytes));
  E.staging_bytes = bytes;
  return FR_HIP_OK;
}

// Copy slices [first, first+n) of a unit (native bytes at `unit`) into
// block `b`, re-tiled. Slices are consecutive in the unit layout.
static int upload_slices(int b, const uint8_t* unit, uint32_t first, uint32_t n) {
  const Layout& l = E.lay[b];
  uint32_t layer0 = first / 513;
  uint64_t off0 = (uint64_t)layer0 * l.layer + (uint64_t)(first % 513) * l.slice;
  uint32_t last = first + n - 1;
  uint64_t off1 = (uint64_t)(last / 513) * l.layer + (uint64_t)(last % 513) * l.slice +
                  ((last % 513) == (uint32_t)kShared ? l.shared_slice : l.slice);
  uint64_t bytes = off1 - off0;
  int rc = ensure_staging(bytes);
  if (rc) return rc;
  CK(hipMemcpyAsync(E.staging, unit + off0, bytes, hipMemcpyHostToDevice, E.stream));
  // retile_kernel addresses slices relative to layer 0 of `src`/`dst`.
  hipLaunchKernelGGL(retile_kernel, dim3(n), dim3(256), 0, E.stream, E.staging - off0, E.block[b],
                     shape_of(l, false), shape_of(l, true), l.layer, first, n);
  CK(hipGetLastError());
  CK(hipStreamSynchronize(E.stream));
  return FR_HIP_OK;
}

int fr_hip_upload(unsigned block, const void* unit, uint64_t len, unsigned hidden, unsigned format) {
  if (!g_open) return FR_HIP_STATE;
  if (block >= (unsigned)kBlocks || !unit) return FR_HIP_INVALID;
  Layout l;
  if (!layout_of(hidden, format, l) || len != l.block) return FR_HIP_INVALID;
  if (E.block[block]) return FR_HIP_STATE;
  CK(hipSetDevice(E.device));
  uint8_t* dev = nullptr;
  if (hipMalloc(&dev, l.block) != hipSuccess) return FR_HIP_IO;
  E.block[block] = dev;
  E.lay[block] = l;
  E.layers[block] = kLayers;
  const uint8_t* src = static_cast<const uint8_t*>(unit);
  // Two layers per step bound the staging buffer.
  for (uint32_t layer = 0; layer < (uint32_t)kLayers; layer += 2) {
    uint32_t nl = layer + 2 <= (uint32_t)kLayers ? 2 : 1;
    int rc = upload_slices((int)block, src, layer * 513, nl * 513);
    if (rc) {
      (void)hipStreamSynchronize(E.stream);
      (void)hipFree(dev);
      E.block[block] = nullptr;
      E.layers[block] = 0;
      return rc;
    }
  }
  return FR_HIP_OK;
}

int fr_hip_reserve(unsigned block, unsigned hidden, unsigned format) {
  if (!g_open) return FR_HIP_STATE;
  if (block >= (unsigned)kBlocks) return FR_HIP_INVALID;
  Layout l;
  if (!layout_of(hidden, format, l)) return FR_HIP_INVALID;
  if (E.block[block]) return FR_HIP_STATE;
  CK(hipSetDevice(E.device));
  uint8_t* dev = nullptr;
  if (hipMalloc(&dev, l.block) != hipSuccess) return FR_HIP_IO;
  if (hipMemsetAsync(dev, 0, l.block, E.stream) != hipSuccess || hipStreamSynchronize(E.stream) != hipSuccess) {
    (void)hipFree(dev);
    return FR_HIP_IO;
  }
  E.block[block] = dev;
  E.lay[block] = l;
  E.layers[block] = kLayers;
  return FR_HIP_OK;
}

int fr_hip_synthetic(unsigned block, unsigned hidden, unsigned format, unsigned layers, uint64_t seed) {
  if (!g_open) return FR_HIP_STATE;
  if (block >= (unsigned)kBlocks || !layers || layers > (unsigned)kLayers) return FR_HIP_INVALID;
  Layout l;
  if (!layout_of(hidden, format, l)) return FR_HIP_INVALID;
  if (E.block[block]) return FR_HIP_STATE;
  CK(hipSetDevice(E.device));
  uint8_t* dev = nullptr;
  if (hipMalloc(&dev, (size_t)layers * l.layer) != hipSuccess) return FR_HIP_IO;
  const uint32_t n = layers * 513;
  hipLaunchKernelGGL(synth_kernel, dim3(n), dim3(256), 0, E.stream, dev, shape_of(l, false), shape_of(l, true),
                     l.layer, 0u, n, seed, (uint32_t)block);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(E.stream) != hipSuccess) {
    (void)hipFree(dev);
    return FR_HIP_IO;
  }
  E.block[block] = dev;
  E.lay[block] = l;
  E.layers[block] = layers;
  return FR_HIP_OK;
}

int fr_hip_debug_read(unsigned block, uint64_t offset, void* out, uint64_t len) {
  if (!g_open) return FR_HIP_STATE;
  if (block >= (unsigned)kBlocks || !out) return FR_HIP_INVALID;
  if (!E.block[block]) return FR_HIP_STATE;
  const uint64_t have = (uint64_t)E.layers[block] * E.lay[block].layer;
  if (offset > have || len > have - offset) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  CK(hipStreamSynchronize(E.stream));
  CK(hipMemcpy(out, E.block[block] + offset, len, hipMemcpyDeviceToHost));
  return FR_HIP_OK;
}

int fr_hip_refresh(unsigned block, const void* unit, unsigned layer, unsigned expert) {
  if (!g_open) return FR_HIP_STATE;
  if (block >= (unsigned)kBlocks || !unit || layer >= (unsigned)kLayers || expert > (unsigned)kShared)
    return FR_HIP_INVALID;
  if (!E.block[block]) return FR_HIP_STATE;
  if (layer >= E.layers[block]) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  return upload_slices((int)block, static_cast<const uint8_t*>(unit), layer * 513 + expert, 1);
}

int fr_hip_release(unsigned block) {
  if (block >= (unsigned)kBlocks) return FR_HIP_INVALID;
  if (!g_open || !E.block[block]) return FR_HIP_STATE;
  (void)hipSetDevice(E.device);
  (void)hipStreamSynchronize(E.stream);
  (void)hipFree(E.block[block]);
  E.block[block] = nullptr;
  E.layers[block] = 0;
  return FR_HIP_OK;
}

size_t fr_hip_plan_bytes(unsigned burst, unsigned hidden) { return plan_capacity(burst, hidden); }

int fr_hip_plan(const fr_hip_request* req, void* plan, size_t cap, size_t* used, unsigned* grid) {
  if (!g_open) return FR_HIP_STATE;
  return build_plan(req, static_cast<uint8_t*>(plan), cap, used, grid);
}

int fr_hip_launch(const void* host_plan, const void* device_plan, void* stream) {
  if (!g_open) return FR_HIP_STATE;
  if (!host_plan || !device_plan) return FR_HIP_INVALID;
  const PlanHeader& H = *static_cast<const PlanHeader*>(host_plan);
  if (!H.burst || H.burst > (unsigned)kMaxBurst) return FR_HIP_INVALID;
  if (H.kind == KIND_LAYER ? !H.ntA || !H.ntB || H.grid != H.ntA + H.ntB
                           : (H.kind != KIND_DECODE && H.kind != KIND_DECODE_ROWS && H.kind != KIND_DECODE_SPLIT &&
                              H.kind != KIND_DECODE_BURST) ||
                                 !H.grid || !decode_table_ok(H))
    return FR_HIP_INVALID;
  return launch(static_cast<const uint8_t*>(device_plan), H, H.grid,
                stream ? static_cast<hipStream_t>(stream) : E.stream);
}

int fr_hip_launch_static(const void* host_plan, const void* device_plan, float* device_y, unsigned* device_status,
                         void* stream) {
  if (!g_open) return FR_HIP_STATE;
  if (!host_plan || !device_plan || !device_y || !device_status) return FR_HIP_INVALID;
  const PlanHeader& H = *static_cast<const PlanHeader*>(host_plan);
  // Plans this variant runs: one token, decode kernels, units within the
  // static scratch.
  if (H.kind != KIND_DECODE && H.kind != KIND_DECODE_ROWS && H.kind != KIND_DECODE_SPLIT) return FR_HIP_UNSUPPORTED;
  if (H.mode != MODE_F32) return FR_HIP_UNSUPPORTED;   // the static array holds float partials
  if (H.kind == KIND_DECODE_SPLIT && H.pad != 2 && H.pad != 4) return FR_HIP_INVALID;
  const unsigned items = H.kind == KIND_DECODE_SPLIT ? H.npairs * H.pad : H.npairs;
  if (H.burst != 1 || items > kStaticUnits || !H.hidden || H.hidden > (unsigned)kMaxHidden) return FR_HIP_UNSUPPORTED;
  if (!H.grid || H.grid > (unsigned)kDecodeGridMax || H.grid > items || H.ngroups != H.burst || !decode_table_ok(H))
    return FR_HIP_INVALID;
  if (H.kind == KIND_DECODE_ROWS && (H.pad & ~kComboShared) > COMBO_Q4_0) return FR_HIP_INVALID;
  if (!E.static_scratch) return FR_HIP_STATE;
  CK(hipSetDevice(E.device));
  Scratch S = {};   // no engine buffers, no host outputs
  S.wgpart = E.static_scratch + kStaticHead;
  S.ustride = kStaticUnits;
  S.ystat = reinterpret_cast<uint32_t*>(device_status);
  S.yout = device_y;
  S.dstat = reinterpret_cast<uint32_t*>(E.static_scratch);
  if (!launch_decode(static_cast<const uint8_t*>(device_plan), H, H.grid, S,
                     stream ? static_cast<hipStream_t>(stream) : E.stream, nullptr))
    return FR_HIP_IO;
  CK(hipGetLastError());
  return FR_HIP_OK;
}

int fr_hip_last_output(void* stream, float* y, size_t count, unsigned* status) {
  if (!g_open) return FR_HIP_STATE;
  if (count > (size_t)kMaxBurst * kMaxHidden) return FR_HIP_INVALID;
  return fetch_output(stream ? static_cast<hipStream_t>(stream) : E.stream, count, y, status);
}

// One run() call's launch; `layer` forces the layer kernel (the plan is
// built with the decode kernels switched off).
double now_ns() {
  return (double)std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

// One attempt of fr_hip_run; adds its plan, enqueue, wait and (with
// phase events) GPU times to ph.
int run_once(const fr_hip_request* req, float* y, bool layer, unsigned* status_out, double (&ph)[FR_HIP_PHASES]) {
  size_t used = 0;
  unsigned grid = 0;
  const double t0 = now_ns();
  const bool no_decode = E.no_decode;
  E.no_decode = no_decode || layer;
  int rc = build_plan(req, E.plan_host, E.plan_cap, &used, &grid);
  E.no_decode = no_decode;
  if (rc) return rc;
  const double t1 = now_ns();
  const bool events = E.phase_events;
  if (events) CK(hipEventRecord(E.pev0, E.stream));
  const PlanHeader& H = *reinterpret_cast<const PlanHeader*>(E.plan_host);
  // The plan (with x) is staged into device memory by a copy kernel, then
  // the launch, then one wait. On the decode path decode_reduce writes y and
  // its status words to mapped host memory, so no copy out is needed; the
  // layer kernel's outputs are copied back. No events on this path
  // (fr_hip_timing times launches on request).
  {
    const unsigned words = (unsigned)((used + 15) / 16);
    hipLaunchKernelGGL(stage_plan, dim3((words + 63) / 64), dim3(64), 0, E.stream, E.plan_mapped,
                       reinterpret_cast<uint4*>(E.plan_dev), words);
  }
  const bool decode = H.kind == KIND_DECODE || H.kind == KIND_DECODE_ROWS || H.kind == KIND_DECODE_SPLIT ||
                      H.kind == KIND_DECODE_BURST;
  rc = launch(E.plan_dev, H, grid, E.stream, decode);
  if (rc) return rc;
  if (events) CK(hipEventRecord(E.pev1, E.stream));
  const double t2 = now_ns();
  const size_t count = (size_t)H.burst * H.hidden;
  unsigned status = 0;
  if (decode) {
    CK(hipStreamSynchronize(E.stream));
    const size_t words = (size_t)H.burst * (kMaxHidden / kReducePositions);
    for (size_t i = 0; i < words; ++i) status |= __atomic_load_n(E.hstat_host + i, __ATOMIC_RELAXED);
  } else {
    rc = fetch_output(E.stream, count, nullptr, &status);
    if (rc) return rc;
  }
  ++E.sample.runs;
  *status_out = status;
  if (!status) memcpy(y, decode ? E.hy_host : reinterpret_cast<const float*>(E.out_host + 4), count * sizeof(float));
  const double t3 = now_ns();
  ph[FR_HIP_PHASE_PLAN] += t1 - t0;
  ph[FR_HIP_PHASE_ENQUEUE] += t2 - t1;
  ph[FR_HIP_PHASE_WAIT] += t3 - t2;
  float ms = 0.f;
  if (events && hipEventElapsedTime(&ms, E.pev0, E.pev1) == hipSuccess) ph[FR_HIP_PHASE_GPU] += (double)ms * 1e6;
  return FR_HIP_OK;
}

int fr_hip_run(const fr_hip_request* req, float* y) {
  if (!g_open) return FR_HIP_STATE;
  if (!req || !y) return FR_HIP_INVALID;
  const double start = now_ns();
  CK(hipSetDevice(E.device));
  unsigned status = 0;
  double ph[FR_HIP_PHASES] = {};
  int rc = run_once(req, y, false, &status, ph);
  // A ref-q8 decode launch that met a weight the reference rounds in float
  // (and nothing else) is run again on the layer kernel.
  if (!rc && status == kErrInexact) rc = run_once(req, y, true, &status, ph);
  if (rc) return rc;
  ph[FR_HIP_PHASE_TOTAL] = now_ns() - start;
  ph[FR_HIP_PHASE_OVERHEAD] = ph[FR_HIP_PHASE_TOTAL] - ph[FR_HIP_PHASE_GPU];
  memcpy(E.phase, ph, sizeof(ph));
  ++E.phase_runs;
  if (status & kErrTimeout) return FR_HIP_IO;
  if (status) return FR_HIP_NUMERIC;   // y is written only on success: untouched on failure
  return FR_HIP_OK;
}

size_t fr_hip_batch_plan_bytes(unsigned tokens, unsigned hidden) { return batch_capacity(tokens, hidden); }

int fr_hip_batch_plan(const fr_hip_batch* req, void* plan, size_t cap, size_t* used) {
  if (!g_open) return FR_HIP_STATE;
  return build_batch(req, static_cast<uint8_t*>(plan), cap, used);
}

int fr_hip_batch_launch(const void* host_plan, const void* device_plan, void* stream) {
  if (!g_open) return FR_HIP_STATE;
  if (!host_plan || !device_plan) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  return batch_launch(static_cast<const uint8_t*>(device_plan), *static_cast<const BatchHeader*>(host_plan),
                      stream ? static_cast<hipStream_t>(stream) : E.stream);
}

int fr_hip_batch_output(void* stream, float* y, size_t count, unsigned* status) {
  if (!g_open) return FR_HIP_STATE;
  return batch_output(stream ? static_cast<hipStream_t>(stream) : E.stream, y, count, status);
}

int fr_hip_run_batch(const fr_hip_batch* req, float* y) {
  if (!g_open) return FR_HIP_STATE;
  if (!req || !y) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  if (req->tokens > (unsigned)kMaxBatchTokens) return FR_HIP_INVALID;
  const size_t need = batch_capacity(req->tokens, req->hidden);
  if (need > E.bplan_cap) {
    (void)hipFree(E.bplan_dev);
    (void)hipHostFree(E.bplan_host);
    E.bplan_dev = nullptr;
    E.bplan_host = nullptr;
    E.bplan_cap = 0;
    CK(hipMalloc(&E.bplan_dev, need));
    CK(hipHostMalloc(reinterpret_cast<void**>(&E.bplan_host), need, hipHostMallocDefault));
    E.bplan_cap = need;
  }
  size_t used = 0;
  int rc = build_batch(req, E.bplan_host, E.bplan_cap, &used);
  if (rc) return rc;
  const BatchHeader& H = *reinterpret_cast<const BatchHeader*>(E.bplan_host);
  CK(hipMemcpyAsync(E.bplan_dev, E.bplan_host, used, hipMemcpyHostToDevice, E.stream));
  CK(hipEventRecord(E.ev0, E.stream));
  rc = batch_launch(E.bplan_dev, H, E.stream);
  if (rc) return rc;
  CK(hipEventRecord(E.ev1, E.stream));
  unsigned status = 0;
  rc = batch_output(E.stream, nullptr, 0, &status);
  if (rc) return rc;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, E.ev0, E.ev1) == hipSuccess) E.sample.last_kernel_ns = ms * 1e6;
  ++E.sample.runs;
  if (status) return FR_HIP_NUMERIC;
  // y is written only on success: untouched on failure.
  CK(hipMemcpy(y, E.by, (size_t)H.tokens * H.hidden * sizeof(float), hipMemcpyDeviceToHost));
  return FR_HIP_OK;
}

int fr_hip_timing(unsigned launches) {
  if (!g_open) return FR_HIP_STATE;
  CK(hipSetDevice(E.device));
  if (launches > E.timed_cap) {
    for (unsigned i = 0; i < 3 * E.timed_cap; ++i) (void)hipEventDestroy(E.tev[i]);
    free(E.tev);
    E.tev = static_cast<hipEvent_t*>(calloc(3 * (size_t)launches, sizeof(hipEvent_t)));
    E.timed_cap = 0;
    if (!E.tev) return FR_HIP_IO;
    for (unsigned i = 0; i < 3 * launches; ++i) CK(hipEventCreate(&E.tev[i]));
    E.timed_cap = launches;
  }
  E.timed = 0;
  E.timing = launches > 0;
  return FR_HIP_OK;
}

int fr_hip_timing_read(double* main_ms, double* total_ms, unsigned* launches) {
  if (!g_open) return FR_HIP_STATE;
  if (!main_ms || !total_ms || !launches) return FR_HIP_INVALID;
  *main_ms = *total_ms = 0.0;
  for (unsigned i = 0; i < E.timed; ++i) {
    float a = 0.f, b = 0.f;
    CK(hipEventSynchronize(E.tev[3 * i + 2]));
    CK(hipEventElapsedTime(&a, E.tev[3 * i], E.tev[3 * i + 1]));
    CK(hipEventElapsedTime(&b, E.tev[3 * i], E.tev[3 * i + 2]));
    *main_ms += a;
    *total_ms += b;
  }
  *launches = E.timed;
  E.timing = false;
  return FR_HIP_OK;
}

int fr_hip_sample_get(fr_hip_sample* out) {
  if (!out) return FR_HIP_INVALID;
  *out = E.sample;
  return FR_HIP_OK;
}

int fr_hip_phase_events(int on) {
  if (!g_open) return FR_HIP_STATE;
  E.phase_events = on != 0;
  return FR_HIP_OK;
}

int fr_hip_phase_get(double* ns, uint64_t* runs) {
  if (!g_open) return FR_HIP_STATE;
  if (!ns) return FR_HIP_INVALID;
  memcpy(ns, E.phase, sizeof(E.phase));
  if (runs) *runs = E.phase_runs;
  return FR_HIP_OK;
}

int fr_hip_route(unsigned flags) {
  if (!g_open) return FR_HIP_STATE;
  if (flags & ~(unsigned)(FR_HIP_ROUTE_NO_DECODE | FR_HIP_ROUTE_NO_BURST | FR_HIP_ROUTE_BURST)) return FR_HIP_INVALID;
  if ((flags & FR_HIP_ROUTE_NO_BURST) && (flags & FR_HIP_ROUTE_BURST)) return FR_HIP_INVALID;
  E.no_decode = (flags & FR_HIP_ROUTE_NO_DECODE) != 0;
  E.no_burst = (flags & FR_HIP_ROUTE_NO_BURST) != 0;
  E.force_burst = (flags & FR_HIP_ROUTE_BURST) != 0;
  return FR_HIP_OK;
}

int fr_hip_stream_probe(const void* device_pieces, unsigned count, unsigned threads, unsigned depth,
                        void* device_sink, void* stream) {
  if (!g_open) return FR_HIP_STATE;
  if (!device_pieces || !device_sink || !count || count > (1u << 20) || !threads || threads > 1024 || threads % 64)
    return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : E.stream;
  const uint64_t* p = static_cast<const uint64_t*>(device_pieces);
  uint32_t* k = static_cast<uint32_t*>(device_sink);
  switch (depth) {
    case 1: hipLaunchKernelGGL(stream_probe<1>, dim3(count), dim3(threads), 0, s, p, k); break;
    case 2: hipLaunchKernelGGL(stream_probe<2>, dim3(count), dim3(threads), 0, s, p, k); break;
    case 4: hipLaunchKernelGGL(stream_probe<4>, dim3(count), dim3(threads), 0, s, p, k); break;
    case 8: hipLaunchKernelGGL(stream_probe<8>, dim3(count), dim3(threads), 0, s, p, k); break;
    default: return FR_HIP_INVALID;
  }
  CK(hipGetLastError());
  return FR_HIP_OK;
}

static int debug_upload(const void* bytes, size_t n, uint8_t** dev) {
  CK(hipMalloc(dev, n ? n : 1));
  CK(hipMemcpy(*dev, bytes, n, hipMemcpyHostToDevice));
  return FR_HIP_OK;
}

int fr_hip_debug_dequant(unsigned type, const void* row, unsigned n, float* out) {
  if (!g_open) return FR_HIP_STATE;
  if (!row || !out || !n || n % 64 || n > (unsigned)kMaxHidden) return FR_HIP_INVALID;
  if (type != TQ4_K && type != TQ8_0 && type != TMXFP4 && type != TQ4_0) return FR_HIP_INVALID;
  if (type == TQ4_K && n % 256) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  // Re-tile the row as row 0 of a gate block of a one-slice layout.
  size_t rb = row_bytes(type, n);
  uint8_t *src = nullptr, *dst = nullptr;
  float* dout = nullptr;
  uint32_t* st = nullptr;
  int rc = debug_upload(row, rb, &src);
  if (rc) return rc;
  CK(hipMalloc(&dst, rb));
  CK(hipMalloc(&dout, n * sizeof(float)));
  CK(hipMalloc(&st, sizeof(uint32_t)));
  CK(hipMemset(st, 0, sizeof(uint32_t)));
  SliceShape s = {n, type, TQ8_0, (uint32_t)rb * kNeurons, 0, (uint32_t)rb};
  // Gather through the same re-tile mapping, one row only.
  hipLaunchKernelGGL(debug_retile_row, dim3(1), dim3(256), 0, E.stream, s, src, dst, (uint32_t)rb);
  hipLaunchKernelGGL(debug_decode_rows, dim3(1), dim3(64), 0, E.stream, (uint8_t)type, dst, n, dout, st);
  CK(hipGetLastError());
  CK(hipStreamSynchronize(E.stream));
  uint32_t status = 0;
  CK(hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost));
  CK(hipMemcpy(&status, st, sizeof(status), hipMemcpyDeviceToHost));
  (void)hipFree(src);
  (void)hipFree(dst);
  (void)hipFree(dout);
  (void)hipFree(st);
  return status ? FR_HIP_NUMERIC : FR_HIP_OK;
}

int fr_hip_debug_dequant_down(unsigned format, const void* down, unsigned hidden, float* out) {
  if (!g_open) return FR_HIP_STATE;
  Layout l;
  if (!down || !out || !layout_of(hidden, format, l)) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  uint8_t *src = nullptr, *dst = nullptr;
  float* dout = nullptr;
  uint32_t* st = nullptr;
  int rc = debug_upload(down, l.down, &src);
  if (rc) return rc;
  CK(hipMalloc(&dst, l.down));
  CK(hipMalloc(&dout, (size_t)hidden * 32 * sizeof(float)));
  CK(hipMalloc(&st, sizeof(uint32_t)));
  CK(hipMemset(st, 0, sizeof(uint32_t)));
  hipLaunchKernelGGL(debug_retile_down, dim3(1), dim3(256), 0, E.stream, (uint8_t)l.dn, hidden, src, dst, (uint32_t)l.down);
  unsigned threads = l.dn == TQ4_KT ? hidden / 256 * 64 : hidden;
  hipLaunchKernelGGL(debug_decode_down, dim3((threads + 255) / 256), dim3(256), 0, E.stream, (uint8_t)l.dn, dst,
                     hidden, dout, st);
  CK(hipGetLastError());
  CK(hipStreamSynchronize(E.stream));
  uint32_t status = 0;
  CK(hipMemcpy(out, dout, (size_t)hidden * 32 * sizeof(float), hipMemcpyDeviceToHost));
  CK(hipMemcpy(&status, st, sizeof(status), hipMemcpyDeviceToHost));
  (void)hipFree(src);
  (void)hipFree(dst);
  (void)hipFree(dout);
  (void)hipFree(st);
  return status ? FR_HIP_NUMERIC : FR_HIP_OK;
}

static int debug_quantize_run(const float* x, unsigned n, float* out, bool regs) {
  if (!g_open) return FR_HIP_STATE;
  if (!x || !out || !n || (n % 64 && (regs || n != 32))) return FR_HIP_INVALID;
  CK(hipSetDevice(E.device));
  float* d = nullptr;
  CK(hipMalloc(&d, n * sizeof(float)));
  CK(hipMemcpy(d, x, n * sizeof(float), hipMemcpyHostToDevice));
  if (regs) hipLaunchKernelGGL(debug_quantize_regs, dim3((n / 64 + 63) / 64), dim3(64), 0, E.stream, d, n / 64);
  else if (n == 32) hipLaunchKernelGGL(debug_quantize32, dim3(1), dim3(64), 0, E.stream, d, 1u);
  else hipLaunchKernelGGL(debug_quantize, dim3((n / 64 + 63) / 64), dim3(64), 0, E.stream, d, n / 64);
  CK(hipGetLastError());
  CK(hipStreamSynchronize(E.stream));
  CK(hipMemcpy(out, d, n * sizeof(float), hipMemcpyDeviceToHost));
  (void)hipFree(d);
  return FR_HIP_OK;
}

int fr_hip_debug_quantize(const float* x, unsigned n, float* out) { return debug_quantize_run(x, n, out, false); }

int fr_hip_debug_quantize8(const float* x, unsigned n, unsigned group, int8_t* q, float* d, int16_t* s) {
  if (!g_open) return FR_HIP_STATE;
  const bool xg = group == 256 && n && n % 256 == 0 && n <= (unsigned)kMaxHidden && s;
  if (!x || !q || !d || !(xg || (group == 32 && n == 32))) return FR_HIP_INVALID;
  if (hipSetDevice(E.device) != hipSuccess) return FR_HIP_IO;
  // One buffer: x, then the codes, the scales and the sums.
  const size_t xb = n * sizeof(float), qb = n, db = n / group * sizeof(float), sb = n / 32 * sizeof(int16_t);
  const size_t qo = xb, dof = (qo + qb + 15) & ~(size_t)15, so = (dof + db + 15) & ~(size_t)15;
  uint8_t* buf = nullptr;
  if (hipMalloc(&buf, so + sb) != hipSuccess) return FR_HIP_IO;
  int rc = FR_HIP_OK;
  if (hipMemcpy(buf, x, xb, hipMemcpyHostToDevice) != hipSuccess) rc = FR_HIP_IO;
  if (!rc) {
    float* dx = reinterpret_cast<float*>(buf);
    int8_t* dq = reinterpret_cast<int8_t*>(buf + qo);
    float* dd = reinterpret_cast<float*>(buf + dof);
    int16_t* ds = reinterpret_cast<int16_t*>(buf + so);
    if (xg) hipLaunchKernelGGL(debug_quantize8_x, dim3(1), dim3(kDecodeThreads), 0, E.stream, dx, n, dq, dd, ds);
    else hipLaunchKernelGGL(debug_quantize8_h, dim3(1), dim3(64), 0, E.stream, dx, dq, dd);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(E.stream) != hipSuccess ||
        hipMemcpy(q, dq, qb, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(d, dd, db, hipMemcpyDeviceToHost) != hipSuccess ||
        (xg && hipMemcpy(s, ds, sb, hipMemcpyDeviceToHost) != hipSuccess))
      rc = FR_HIP_IO;
  }
  (void)hipFree(buf);
  return rc;
}
int fr_hip_debug_quantize64(const float* x, unsigned n, float* out) { return debug_quantize_run(x, n, out, true); }

int fr_hip_debug_partials(unsigned first, unsigned count, float* out) {
  if (!g_open) return FR_HIP_STATE;
  if (!out || !count || first + count > (unsigned)kMaxDecodeItems || first + count < first) return FR_HIP_INVALID;
  if (hipSetDevice(E.device) != hipSuccess || hipStreamSynchronize(E.stream) != hipSuccess) return FR_HIP_IO;
  // Position block pb of the items sits at pb * kMaxDecodeItems + item (16
  // floats each, partial_index); copy each block's run of items.
  std::vector<float> blk((size_t)count * 16);
  for (unsigned pb = 0; pb < (unsigned)kMaxHidden / 16; ++pb) {
    const float* src = E.wgpart + ((size_t)pb * kMaxDecodeItems + first) * 16;
    if (hipMemcpy(blk.data(), src, blk.size() * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) return FR_HIP_IO;
    for (unsigned i = 0; i < count; ++i)
      for (unsigned k = 0; k < 16; ++k) {
        const unsigned p = 16 * pb + k;
        const unsigned w = p >> 9, hh = (p >> 8) & 1, l = (p >> 2) & 63, cc = p & 3;   // decode_column
        out[(size_t)i * kMaxHidden + 256 * (2 * w + (l >> 5)) + 8 * (l & 31) + 4 * hh + cc] = blk[16 * i + k];
      }
  }
  return FR_HIP_OK;
}

int fr_hip_debug_quantize_staged(const float* x, unsigned n, unsigned form, float* out, double* sums) {
  if (!g_open) return FR_HIP_STATE;
  if (!x || !out || form > 2) return FR_HIP_INVALID;
  if (form == 2 ? n != 32 : (!sums || !n || n % 64 || n > (unsigned)kMaxHidden)) return FR_HIP_INVALID;
  if (hipSetDevice(E.device) != hipSuccess) return FR_HIP_IO;
  // One buffer: x, the rebuilt values, the sums, the status word.
  const size_t xb = (size_t)n * sizeof(float), ob = xb, sb = (size_t)(n / 32) * sizeof(double);
  uint8_t* buf = nullptr;
  if (hipMalloc(&buf, xb + ob + sb + 16) != hipSuccess) return FR_HIP_IO;
  float* dx = reinterpret_cast<float*>(buf);
  float* dout = reinterpret_cast<float*>(buf + xb);
  double* dsum = reinterpret_cast<double*>(buf + xb + ob);
  uint32_t* dst = reinterpret_cast<uint32_t*>(buf + xb + ob + sb);
  uint32_t status = 0;
  int rc = FR_HIP_OK;
  if (hipMemcpy(dx, x, xb, hipMemcpyHostToDevice) != hipSuccess || hipMemset(dst, 0, 4) != hipSuccess) rc = FR_HIP_IO;
  if (!rc) {
    hipLaunchKernelGGL(debug_quantize_staged, dim3(1), dim3(kDecodeThreads), 0, E.stream, dx, n, form, dout, dsum, dst);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(E.stream) != hipSuccess ||
        hipMemcpy(out, dout, ob, hipMemcpyDeviceToHost) != hipSuccess ||
        (form != 2 && hipMemcpy(sums, dsum, sb, hipMemcpyDeviceToHost) != hipSuccess) ||
        hipMemcpy(&status, dst, 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = FR_HIP_IO;
  }
  (void)hipFree(buf);
  if (!rc && status) rc = FR_HIP_NUMERIC;
  return rc;
}

}  // extern "C"
