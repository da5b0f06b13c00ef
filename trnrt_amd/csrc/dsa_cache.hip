// Quantise-on-write into the paged FP8 caches for gfx950: the cache-store step before the DSA path
// (trnrt/models/decoder.py:481-486 `_store`, called for the latent rows and the indexer-key rows at
// trnrt/models/mla.py:445-446), with the per-token scale of this build's cache format:
//
//   scaled form:    s = max(absmax(x_row), 1e-30) / 448,  cache[slot] = e4m3fn(clamp(x_row / s, +-fp8_max)),
//                   scale[slot] = s
//   reference form: cache[slot] = e4m3fn(clamp(x_row, +-fp8_max)),  scale[slot] = 1 (when a scale array is given)
//
// in fp32 with a correctly rounded division and round-to-nearest-even into e4m3fn (v_cvt_pk_fp8_f32), which is
// torch's float -> float8_e4m3fn cast. One wave per row: each lane converts groups of 8 values (16 bytes of bf16 or
// 32 of fp32 in, 8 bytes out), the row's absmax is a wave reduction, and lane 0 writes the scale. A row whose slot
// is outside [0, num_slots) is not written.
#include "dsa_common.h"

namespace dsa {

constexpr int CW_WAVES = 4;              // rows per workgroup
constexpr int CW_GPL = 2;                // groups of 8 values per lane: rows up to 64 x 8 x 2 = 1024 values
constexpr float CW_FP8_MAX = 448.0f;     // the e4m3fn maximum (the scale's target)

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float (&v)[8]) {  // bf16 bits
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

template <typename T, bool SCALED>
__global__ __launch_bounds__(CW_WAVES * WAVE) void cache_write_kernel(const T* __restrict__ x,
                                                                      const int64_t* __restrict__ slots,
                                                                      uint8_t* __restrict__ cache,
                                                                      float* __restrict__ cscale, int n_rows, int W,
                                                                      long num_slots, float fp8_max) {
  const int row = blockIdx.x * CW_WAVES + (int)(threadIdx.x / WAVE);
  const int lane = threadIdx.x & (WAVE - 1);
  if (row >= n_rows) return;  // wave-uniform
  const long slot = slots[row];
  if (slot < 0 || slot >= num_slots) return;  // wave-uniform
  const int G = W / 8;
  const T* xr = x + (size_t)row * W;
  float v[CW_GPL][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CW_GPL; ++i) {
    const int g = lane + WAVE * i;
    load8<T>(xr + 8 * min(g, G - 1), v[i]);  // in range whatever the lane; lanes past the row add nothing
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = g < G ? fmaxf(amax, fabsf(v[i][e])) : amax;
  }
  float s = 1.0f;
  if (SCALED) s = fmaxf(wave_max(amax), 1e-30f) / CW_FP8_MAX;
  uint8_t* cr = cache + (size_t)slot * W;
#pragma unroll
  for (int i = 0; i < CW_GPL; ++i) {
    const int g = lane + WAVE * i;
    if (g >= G) break;
    float q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = fminf(fmaxf(SCALED ? v[i][e] / s : v[i][e], -fp8_max), fp8_max);
    int lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
    *reinterpret_cast<uint2*>(cr + 8 * g) = make_uint2((uint32_t)lo, (uint32_t)hi);
  }
  if (cscale && lane == 0) cscale[slot] = s;
}

template <typename T>
static hipError_t launch_cache_write_t(const T* x, const int64_t* slots, uint8_t* cache, float* cscale, int n_rows,
                                       int W, long num_slots, int scaled, float fp8_max, hipStream_t s) {
  const dim3 grid((n_rows + CW_WAVES - 1) / CW_WAVES);
  if (scaled)
    return launch("cache_write_kernel", cache_write_kernel<T, true>, grid, dim3(CW_WAVES * WAVE), s, x, slots, cache,
                  cscale, n_rows, W, num_slots, fp8_max);
  return launch("cache_write_kernel", cache_write_kernel<T, false>, grid, dim3(CW_WAVES * WAVE), s, x, slots, cache,
                cscale, n_rows, W, num_slots, fp8_max);
}

bool cache_write_width_ok(int W) { return W >= 8 && W % 8 == 0 && W <= WAVE * 8 * CW_GPL; }

hipError_t launch_cache_write(const void* x, int x_fp32, const int64_t* slots, uint8_t* cache, float* cscale,
                              int n_rows, int W, long num_slots, int scaled, float fp8_max, hipStream_t s) {
  if (x_fp32)
    return launch_cache_write_t(static_cast<const float*>(x), slots, cache, cscale, n_rows, W, num_slots, scaled,
                                fp8_max, s);
  return launch_cache_write_t(static_cast<const uint16_t*>(x), slots, cache, cscale, n_rows, W, num_slots, scaled,
                              fp8_max, s);
}

// GLM's pooled indexer keys, written with the cache (trnrt/models/mla.py:1262-1296 `write_pool_keys` with
// trnrt/models/glm5_next.py:151-160 `pool_keys`): for every written token, its pool's kp cached indexer rows
// [key (Di) | gate logits (Di)] give the pool key
//
//   pk[d] = bf16( sum_t bf16( bf16(softmax_t(g_t[d] + ape[t, d])) * k_t[d] ) )    (softmax over the pool, fp32)
//
// written as kp pieces of Di / kp values, piece i into the slot of the pool's i-th token (a padded row, slot in the
// null page, writes all its pieces into its own slot). One wave per written token, 2 channels per lane (Di = 128).
constexpr int PK_MAXKP = 8;

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float((uint32_t)f32_to_bf16_bits(x) << 16); }

template <bool FP8>
__global__ __launch_bounds__(CW_WAVES * WAVE) void pool_keys_kernel(
    const void* __restrict__ rows, const float* __restrict__ rows_scale, int rows_width, const float* __restrict__ ape,
    const int* __restrict__ positions, const int* __restrict__ table, int table_shared, int table_pages,
    const int64_t* __restrict__ slot_mapping, uint16_t* __restrict__ pool_key, int T, int kp, int page_size,
    long num_slots) {
  constexpr int Di = 128;
  const int row = blockIdx.x * CW_WAVES + (int)(threadIdx.x / WAVE);
  const int lane = threadIdx.x & (WAVE - 1);
  if (row >= T) return;  // wave-uniform
  const long own = slot_mapping[row];
  const bool real = own >= page_size;
  const int pos = positions[row];
  // a pool never straddles a page (page_size % kp == 0), so its tokens' slots (table[p / page_size] page_size +
  // p % page_size for p = pos - pos % kp + t, trnrt/models/mla.py:1262-1274) are the written row's own slot's
  // neighbours: own - pos % kp + t. No dependent table read.
  (void)table, (void)table_shared, (void)table_pages;
  const int off = pos - (pos / kp) * kp;
  long slot[PK_MAXKP];
#pragma unroll
  for (int t = 0; t < PK_MAXKP; ++t) {
    slot[t] = real ? own - off + min(t, kp - 1) : own;
    slot[t] = min(max(slot[t], 0L), num_slots - 1);  // in range whatever the inputs
  }
  // this lane's two channels d = 2 lane, 2 lane + 1 of every token of the pool: key and gate logit
  float k[PK_MAXKP][2], l[PK_MAXKP][2];
#pragma unroll
  for (int t = 0; t < PK_MAXKP; ++t) {
    const size_t base = (size_t)slot[t] * rows_width;
    if (FP8) {
      const uint8_t* r = static_cast<const uint8_t*>(rows) + base;
      const float sc = rows_scale ? rows_scale[slot[t]] : 1.0f;
      const uint16_t kb = *reinterpret_cast<const uint16_t*>(r + 2 * lane);
      const uint16_t gb = *reinterpret_cast<const uint16_t*>(r + Di + 2 * lane);
      const auto kf = __builtin_amdgcn_cvt_pk_f32_fp8(kb, false);
      const auto gf = __builtin_amdgcn_cvt_pk_f32_fp8(gb, false);
      // the reference reads the FP8 rows in the model dtype (bf16), exact for e4m3 values; a per-token scale, when
      // the cache has one, is applied in fp32 and rounded back to bf16
      k[t][0] = bf16_round(kf[0] * sc), k[t][1] = bf16_round(kf[1] * sc);
      l[t][0] = bf16_round(gf[0] * sc), l[t][1] = bf16_round(gf[1] * sc);
    } else {
      const uint16_t* r = static_cast<const uint16_t*>(rows) + base;
      const uint32_t kw = *reinterpret_cast<const uint32_t*>(r + 2 * lane);
      const uint32_t gw = *reinterpret_cast<const uint32_t*>(r + Di + 2 * lane);
      k[t][0] = __uint_as_float(kw << 16), k[t][1] = __uint_as_float(kw & 0xffff0000u);
      l[t][0] = __uint_as_float(gw << 16), l[t][1] = __uint_as_float(gw & 0xffff0000u);
    }
  }
  uint16_t out[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int d = 2 * lane + c;
    float x[PK_MAXKP], m = -INFINITY;
#pragma unroll
    for (int t = 0; t < PK_MAXKP; ++t) {
      x[t] = l[t][c] + ape[min(t, kp - 1) * Di + d];
      if (t < kp) m = fmaxf(m, x[t]);
    }
    float e[PK_MAXKP], sum = 0.0f;
#pragma unroll
    for (int t = 0; t < PK_MAXKP; ++t) {
      e[t] = t < kp ? expf(x[t] - m) : 0.0f;
      sum += e[t];
    }
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < PK_MAXKP; ++t)
      if (t < kp) acc += bf16_round(bf16_round(e[t] / sum) * k[t][c]);
    out[c] = f32_to_bf16_bits(acc);
  }
  // piece i (channels i Di / kp ..) into slot i: this lane's two channels
  const int per = Di / kp;
  const int piece = (2 * lane) / per;
  const long dst = slot[min(piece, PK_MAXKP - 1)];
  *reinterpret_cast<uint32_t*>(pool_key + (size_t)dst * per + (2 * lane - piece * per)) =
      (uint32_t)out[0] | ((uint32_t)out[1] << 16);
}

hipError_t launch_pool_keys(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                            const int* positions, const int* table, int table_shared, int table_pages,
                            const int64_t* slot_mapping, uint16_t* pool_key, int T, int kp, int page_size,
                            long num_slots, hipStream_t s) {
  const dim3 grid((T + CW_WAVES - 1) / CW_WAVES);
  if (rows_fp8)
    return launch("pool_keys_kernel", pool_keys_kernel<true>, grid, dim3(CW_WAVES * WAVE), s, rows, rows_scale,
                  rows_width, ape, positions, table, table_shared, table_pages, slot_mapping, pool_key, T, kp,
                  page_size, num_slots);
  return launch("pool_keys_kernel", pool_keys_kernel<false>, grid, dim3(CW_WAVES * WAVE), s, rows, rows_scale,
                rows_width, ape, positions, table, table_shared, table_pages, slot_mapping, pool_key, T, kp,
                page_size, num_slots);
}

}  // namespace dsa
