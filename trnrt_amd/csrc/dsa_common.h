// Shared device helpers of the gfx950 DSA decode kernels: vector types for the MFMA operands, the OCP e4m3fn ->
// bf16 conversion, the order-preserving integer key of an fp32 score, and wave/block reductions for wave64.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

// Kernel timing for benchmarks: while a KernelTimer is installed on the calling host thread, every kernel this
// library launches takes the next pair of its events, recorded by the runtime at the kernel's own start and end
// (hipExtLaunchKernel), and its name; launches past the supplied pairs are counted but not timed.
struct KernelTimer {
  hipEvent_t* events;  // 2 * pairs events, created by the caller
  int pairs;
  int launched;
  const char* names[32];
};
extern thread_local KernelTimer* g_kernel_timer;

// Launches kernel<<<grid, block, 0, s>>>(args...) (through hipExtLaunchKernel, so an installed KernelTimer can
// time it). Returns the launch status.
template <typename F, typename... Args>
inline hipError_t launch(const char* name, F kernel, dim3 grid, dim3 block, hipStream_t s, Args... args) {
  KernelTimer* t = g_kernel_timer;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (t) {
    if (t->launched < t->pairs) {
      e0 = t->events[2 * t->launched];
      e1 = t->events[2 * t->launched + 1];
    }
    if (t->launched < 32) t->names[t->launched] = name;
    ++t->launched;
  }
  hipExtLaunchKernelGGL(kernel, grid, block, 0, s, e0, e1, 0, args...);
  return hipGetLastError();
}

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

// A 16-byte load that bypasses the caches' retention policy for data read exactly once (streamed cache pages).
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

constexpr float NEG_INF = -1e30f;   // trnrt/models/decoder.py NEG_INF
// The top-k's first-level histogram of a row: 4096 bins (the top 12 bits of the order key), kept in HIST_REPLICAS
// copies that the indexer's workgroups fill in turn (fewer atomics on the same address); readers sum the copies.
constexpr int HIST_BINS = 4096;

// The attention's pooled token form (kpool = 1 << kp_shift > 1; kp_shift 0: the per-token forms): idx holds
// idx_stride selected pools per row, npool [B] each row's complete pools (its tail pool), positions [B] its position.
// tail_apart: the row's tail tokens are not among the kernel's slots but added by the workgroup that holds the row's
// last slot (the split form), so the kpool x idx_stride slots of the selected pools split into whole chunks.
struct PoolForm {
  int kp_shift;
  int idx_stride;
  const int* npool;
  const int* positions;
  int tail_apart;
  int empty_n;         // rows + cnt form: the masked slots a row with cnt 0 attends (0: one)
  const int* n_live;   // null, or one int on the device: rows at or past it are neither computed nor written
};
// The pooled decode step's pool-key write, folded into the pooled layer's launch (dsa_pooled_decode_step): the
// indexer rows cache [slots][rows_width] (e4m3 with a per-slot fp32 scale, or bf16: rows_fp8 0), the pool-position
// bias [kpool][128] fp32 and each row's written token's cache slot.
struct PoolKeyWrite {
  const void* rows;
  const float* rows_scale;
  const float* ape;
  const int64_t* slot_mapping;
  int rows_width;
  int rows_fp8;
};
constexpr int HIST_REPLICAS = 1;
// The first bytes of every decode workspace, at the same offset whatever the batch size: per XCD (8 x 256 words) eight
// 128-byte lines. Word 0 of each line is a copy of the XCD-local barriers' arrival counter (a multiple of 256 between
// calls: each launch adds 256 to every copy); the first line then holds an unused word (zero) and two status words
// that persist across calls until dsa_layer_status clears them: the count of barrier waits that gave up, and the
// count of rows that took the one-launch layer's two-exchange selection. Every other word is zero. The top-k
// histograms (zero between calls) follow. Each arrival adds to every copy and each workgroup polls one, so a copy's
// line takes the polls of 4 of the XCD's 32 workgroups; with two XCDs' counters in one line their polls and
// arrivals queued on each other (measured: 0.6-0.9 us a launch of the one-launch layers), and four or eight copies a
// line of their own took 0.2-0.3 us more off.
constexpr int WS_SYNC_LINES = 8;
constexpr int WS_SYNC_LINE_WORDS = 32;
constexpr int WS_SYNC_WORDS = WS_SYNC_LINE_WORDS * WS_SYNC_LINES;  // per XCD
constexpr int WS_SYNC_BYTES = 8 * 4 * WS_SYNC_WORDS;
constexpr int WS_SYNC_GAVE_UP = 2;
constexpr int WS_SYNC_TWO_EXCHANGE = 3;

// The top-k histograms of a workspace (past the barrier and status words).
__host__ __device__ inline int* ws_hist(void* ws) {
  return reinterpret_cast<int*>(static_cast<char*>(ws) + WS_SYNC_BYTES);
}

// s_waitcnt's immediate for "vector memory count <= n" (expcnt and lgkmcnt left at their maxima, no wait)
__host__ __device__ constexpr int vmcnt_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr float VISIBLE = -5e29f;   // trnrt/kernels/dsa_topk.py:58: scores at or below are not selectable
constexpr int WAVE = 64;

// Two OCP e4m3fn bytes (the low or high 16 bits of `w`) -> two bf16. Every e4m3fn value is exact in bf16, so the
// conversion is exact (v_cvt_scalef32_pk_bf16_fp8 with scale 1).
template <bool HI>
__device__ __forceinline__ bf16x2 fp8x2_to_bf16(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
}

// Eight e4m3fn bytes (two dwords, byte order = element order) -> the 8-element bf16 MFMA operand.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  bf16x2 a = fp8x2_to_bf16<false>(lo), b = fp8x2_to_bf16<true>(lo);
  bf16x2 c = fp8x2_to_bf16<false>(hi), d = fp8x2_to_bf16<true>(hi);
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// Eight bf16 held as four dwords -> the MFMA operand (a bit cast).
// relu of an fp32 value as one integer max on its bits: negative values (sign bit set) are negative integers, so
// they become +0; non-negative values are unchanged (fmaxf would add a NaN-quieting max on every MFMA result)
__device__ __forceinline__ float relu(float x) {
  return __builtin_bit_cast(float, max(__builtin_bit_cast(int, x), 0));
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// fp32 -> bf16 bits, round to nearest even (finite inputs).
// Two fp32 values -> two bf16 (round to nearest even, v_cvt_pk_bf16_f32), a in the low half.
__device__ __forceinline__ uint32_t bf16_pack(float a, float b) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef __bf16 b2v __attribute__((ext_vector_type(2)));
  const f2v v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2v));
}

// max of two fp32 values that are never NaN (scores, maxima) as one v_med3_f32 (the median of a, b and +inf is the
// larger of a and b), without the NaN-quieting that fmaxf adds to each operand
__device__ __forceinline__ float max_nonan(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, INFINITY); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

// Order-preserving key of an fp32 score: a < b (IEEE) <=> key(a) < key(b), -0.0 and +0.0 share a key, and every
// score above VISIBLE has a key > 0, so 0 can stand for "not selectable". NaN is not allowed.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u << 1) == 0) u = 0;  // -0.0 -> +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Cross-lane steps by DPP (data parallel primitives: a lane reads a neighbour's register in the same VALU
// instruction), which cost a few cycles where an LDS-routed shuffle costs a round trip through the LDS pipeline.
// Controls (GFX9): quad_perm [1,0,3,2] = 0xb1, [2,3,0,1] = 0x4e; row_shr:n = 0x110 + n; row_mirror = 0x140,
// row_half_mirror = 0x141; row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = true>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, BOUND_ZERO);
}

// Inclusive prefix sum over the 64 lanes (wrapping uint32 sums, so packed counters add field-wise): Hillis-Steele
// within each row of 16 lanes, then row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then rows 0-1's
// total into rows 2-3 (row_bcast:31). Lanes a DPP step does not write add the old value 0.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  int x = (int)v;
  x += dpp<0x111>(x);
  x += dpp<0x112>(x);
  x += dpp<0x114>(x);
  x += dpp<0x118>(x);
  x += dpp<0x142, 0xa, false>(x);
  x += dpp<0x143, 0xc, false>(x);
  return (uint32_t)x;
}

__device__ __forceinline__ int wave_incl_scan(int v) { return (int)wave_incl_scan_u32((uint32_t)v); }

// Inclusive prefix sum within each row of 16 lanes (the first four steps of the wave scan).
__device__ __forceinline__ int row_incl_scan(int x) {
  x += dpp<0x111>(x);
  x += dpp<0x112>(x);
  x += dpp<0x114>(x);
  x += dpp<0x118>(x);
  return x;
}

// The sum over each row of 16 lanes, in every lane of the row (quad swaps, then half-row and row mirrors).
__device__ __forceinline__ int row_sum(int v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}

// The maximum over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, __int_as_float(dpp<0xb1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x4e>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x141>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x140>(__float_as_int(v))));
  return v;
}

__device__ __forceinline__ float row_sum(float v) {
  v += __int_as_float(dpp<0xb1>(__float_as_int(v)));
  v += __int_as_float(dpp<0x4e>(__float_as_int(v)));
  v += __int_as_float(dpp<0x141>(__float_as_int(v)));
  v += __int_as_float(dpp<0x140>(__float_as_int(v)));
  return v;
}

// The value of the neighbouring lane (lane ^ 1), by a quad permutation.
__device__ __forceinline__ float lane_xor1(float v) { return __int_as_float(dpp<0xb1>(__float_as_int(v))); }

// Wave-wide sum, the same value in every lane (the last lane of the inclusive scan).
__device__ __forceinline__ int wave_sum(int v) {
  return __builtin_amdgcn_readlane((int)wave_incl_scan_u32((uint32_t)v), WAVE - 1);
}

__device__ __forceinline__ float wave_sum(float v) {
  // within rows: quad swaps, half-row and row mirrors; then the four rows' sums
  v += __int_as_float(dpp<0xb1>(__float_as_int(v)));
  v += __int_as_float(dpp<0x4e>(__float_as_int(v)));
  v += __int_as_float(dpp<0x141>(__float_as_int(v)));
  v += __int_as_float(dpp<0x140>(__float_as_int(v)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(dpp<0xb1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x4e>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x141>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp<0x140>(__float_as_int(v))));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp<0xb1>((int)v));
  v = max(v, (uint32_t)dpp<0x4e>((int)v));
  v = max(v, (uint32_t)dpp<0x141>((int)v));
  v = max(v, (uint32_t)dpp<0x140>((int)v));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(r0, r1), max(r2, r3));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)dpp<0xb1>((int)v));
  v = min(v, (uint32_t)dpp<0x4e>((int)v));
  v = min(v, (uint32_t)dpp<0x141>((int)v));
  v = min(v, (uint32_t)dpp<0x140>((int)v));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return min(min(r0, r1), min(r2, r3));
}

// Clamp a page id into the cache (an id outside it reads the null page 0 instead of faulting).
__device__ __forceinline__ int safe_page(int page, int num_pages) {
  return ((unsigned)page < (unsigned)num_pages) ? page : 0;
}

}  // namespace dsa
