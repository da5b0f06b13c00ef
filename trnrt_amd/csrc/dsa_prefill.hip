// Dense (prefill-chunk) lightning indexer for gfx950: the index scores of N queries that share one context's keys
// (the arithmetic of trnrt/kernels/dsa_long_select.py:119-133 `emulate_scores` and trnrt/models/dsa_long.py:74-84
// `scores` with a 2-D key tensor), with per-token FP8 key scales applied after the dot product:
//
//   score[n, p] = scale * k_scale[p] * sum_h w[n, h] * relu(q[n, h, :] . k_fp8[p, :])   for p < npool[n]
//   score[n, p] = NEG_INF                                                               for npool[n] <= p < stride
//
// (relu(a x) = a relu(x) for a = scale * k_scale[p] > 0, so this is dsa_long.scores' w relu(scale q . pk) with
// pk = k_fp8 k_scale.) It is a batched GEMM, (query, head) rows x keys over 128 dims, with a head-reducing epilogue.
// One workgroup = 4 queries (one per wave) x a block of keys, walked in tiles of 32: the workgroup loads a tile's
// 4 KiB of keys coalesced (16 bytes per thread), converts them once to bf16 (exact) into LDS, and every wave
// multiplies its query's 64 heads against them with v_mfma_f32_32x32x16_bf16 (heads as rows: the query operand
// stays in registers for the whole block), so each key byte is read from memory once per 4 queries and converted
// once per workgroup. The bf16 tile is double-buffered (one barrier per tile) and stored with an XOR swizzle (piece
// p of key j at slot 16 j + (p ^ (j & 15))) so the operand reads of 16 lanes hit 16 different bank groups.
//
// Every product is exact in the fp32 accumulator (bf16 x bf16), as in the reference's bf16 matmul; only the fp32
// summation order differs (the reference sums even and odd heads in two accumulators; this sums per lane, then
// across the two lane halves).
#include "dsa_common.h"

namespace dsa {

constexpr int PF_D = 128;
constexpr int PF_TILE = 32;               // keys per tile
constexpr int PF_THREADS = 256;           // 4 waves, one query each
constexpr int PF_QPW = PF_THREADS / WAVE;  // queries per workgroup
constexpr int PF_TILES = 32;              // tiles per workgroup: 1024 keys

// MT: head tiles of 32 (Hi <= 32 MT).
template <int MT>
__global__ __launch_bounds__(PF_THREADS, 2) void indexer_prefill_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint8_t* __restrict__ kcache,
    const float* __restrict__ kscale, const int* __restrict__ npool, float* __restrict__ scores, int N, int Hi, int P,
    int stride, float scale) {
  __shared__ u32x4 kb[2][PF_TILE * 16];  // two bf16 tiles: key j, 16 pieces of 8 dims (swizzled)
  __shared__ int lmax[PF_QPW];
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;  // key column of an MFMA tile / head row of the query operand
  const int h = lane >> 5;  // lane half: dims 16 s + 8 h .. + 7 at step s
  const int n = blockIdx.x * PF_QPW + wave;
  const int nq = min(n, N - 1);  // a wave past N computes a copy of the last query and stores nothing
  const int p_begin = blockIdx.y * PF_TILES * PF_TILE;
  const int p_end = min(p_begin + PF_TILES * PF_TILE, stride);

  int L = min(max(npool[nq], 0), P);
  if (lane == 0) lmax[wave] = L;

  // the query operand (head 32m + j, dims 16 s + 8 h .. + 7 at step s; zero heads past Hi) and head weights in the
  // accumulator layout (register r of head tile m: head 32m + 8(r/4) + 4h + r%4)
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int head = 32 * m + j;
    const uint16_t* qp = q + ((size_t)nq * Hi + min(head, Hi - 1)) * PF_D + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 16 * s);
      qa[m][s] = as_bf16x8(head < Hi ? v : make_uint4(0, 0, 0, 0));
    }
  }
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int head = 32 * m + 8 * (r >> 2) + 4 * h + (r & 3);
      const float x = w[(size_t)nq * Hi + min(head, Hi - 1)];
      wr[m][r] = head < Hi ? x : 0.0f;
    }
  __syncthreads();
  const int wg_L = max(max(lmax[0], lmax[1]), max(lmax[2], lmax[3]));  // keys past every query's count: no MFMA

  // this thread's share of a tile: key t / 8, bytes 16 (t % 8) .. + 15 (coalesced), converted into two pieces
  const int tk = threadIdx.x >> 3, tp = threadIdx.x & 7;
  auto load_tile = [&](int p0) {
    const int key = min(p0 + tk, P - 1);  // in range whatever the block
    return *reinterpret_cast<const uint4*>(kcache + (size_t)key * PF_D + 16 * tp);
  };
  uint4 cur = load_tile(p_begin);
  float* srow = scores + (size_t)n * stride;
  for (int p0 = p_begin, it = 0; p0 < p_end; p0 += PF_TILE, ++it) {
    const uint4 nxt = load_tile(p0 + PF_TILE < p_end ? p0 + PF_TILE : p0);  // the next tile's loads fly meanwhile
    const float ksc = kscale[min(p0 + j, P - 1)];
    // convert and store: dims 16 tp .. +15 of key tk are pieces 2 tp, 2 tp + 1
    u32x4* tile = kb[it & 1];
    {
      const bf16x8 lo = fp8x8_to_bf16x8(cur.x, cur.y), hi = fp8x8_to_bf16x8(cur.z, cur.w);
      tile[16 * tk + ((2 * tp) ^ (tk & 15))] = __builtin_bit_cast(u32x4, lo);
      tile[16 * tk + ((2 * tp + 1) ^ (tk & 15))] = __builtin_bit_cast(u32x4, hi);
    }
    cur = nxt;
    __syncthreads();  // the tile is in LDS; the other buffer is free (every wave finished the previous tile)
    const int pos = p0 + j;
    if (p0 < wg_L) {
      f32x16 acc[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int pc = 2 * s + h;
        const bf16x8 kbv = __builtin_bit_cast(bf16x8, tile[16 * j + (pc ^ (j & 15))]);
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kbv, acc[m], 0, 0, 0);
      }
      float part = 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], fmaxf(acc[m][r], 0.0f), part);
      part += __shfl_xor(part, 32, WAVE);
      const float v = pos < L ? part * (ksc * scale) : NEG_INF;
      if (n < N && h == 0 && pos < p_end) srow[pos] = v;
    } else if (n < N && h == 0 && pos < p_end) {
      srow[pos] = NEG_INF;
    }
  }
}

template <int MT>
static hipError_t launch_prefill_mt(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                    const int* npool, float* scores, int N, int Hi, int P, int stride, float scale,
                                    hipStream_t s) {
  const dim3 grid((N + PF_QPW - 1) / PF_QPW, (stride + PF_TILES * PF_TILE - 1) / (PF_TILES * PF_TILE));
  return launch("indexer_prefill_kernel", indexer_prefill_kernel<MT>, grid, dim3(PF_THREADS), s, q, w, k, ks, npool,
                scores, N, Hi, P, stride, scale);
}

hipError_t launch_indexer_prefill(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                  const int* npool, float* scores, int N, int Hi, int P, int stride, float scale,
                                  hipStream_t s) {
  if (Hi <= 32) return launch_prefill_mt<1>(q, w, k, ks, npool, scores, N, Hi, P, stride, scale, s);
  return launch_prefill_mt<2>(q, w, k, ks, npool, scores, N, Hi, P, stride, scale, s);
}

}  // namespace dsa
