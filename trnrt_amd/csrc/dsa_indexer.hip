// Decode lightning indexer for gfx950: scores of every cached token of every decode row, read once from the paged
// FP8 indexer-key cache (the arithmetic of trnrt/kernels/dsa_index.py:44-50 and trnrt/models/dsa_long.py:74-84 with
// per-token FP8 dequantisation applied after the dot product, which is exact in value because relu(s x) = s relu(x)
// for a scale s > 0):
//
//   score[b, t] = k_scale[slot] * sum_h w[b, h] * relu(q[b, h, :] . k_fp8[slot, :])   (+ cand[b, t])
//
// One wave scores 32 keys per MFMA tile: D[head, key] = Q[head, :] . K[key, :] with v_mfma_f32_32x32x16_bf16, the
// query heads as rows (A operand, held in registers for the wave's whole run) and the keys as columns (B operand,
// e4m3fn bytes converted to bf16 in registers: every e4m3 value is exact in bf16, so each product is exact in the
// fp32 accumulator, as in the reference's "bf16 x bf16 accumulated in fp32", dsa_index.py:13-16). The contraction
// order over the 128 dims is permuted so that each lane reads 64 contiguous key bytes: lane (key j, half h) supplies
// dims 64h + 8s .. 64h + 8s + 7 at MFMA step s, and the query operand uses the same permutation.
//
// The MFMA result leaves lane (j, h) with 16 heads of key j per head tile, so the weighted relu head sum is 16 fused
// multiply-adds per tile in registers plus one exchange between the two lane halves. Only [B, score_stride] fp32
// scores leave the chip: 4 bytes per key against the key's 132.
#include "dsa_common.h"

namespace dsa {

constexpr int IDX_D = 128;        // index_head_dim
constexpr int IDX_TILE = 32;      // keys per MFMA tile
constexpr int IDX_THREADS = 256;  // 4 waves per workgroup
constexpr int IDX_WAVES = IDX_THREADS / WAVE;

struct KeyTile {
  uint4 v[4];  // 64 key bytes of this lane
  float scale;
};

// MT: query-head tiles of 32 (Hi <= 32 MT). Each wave scores `tiles_per_wave` consecutive 32-key tiles of one row.
template <int MT>
__global__ __launch_bounds__(IDX_THREADS) void indexer_decode_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint8_t* __restrict__ kcache,
    const float* __restrict__ kscale, const int* __restrict__ table, const int* __restrict__ ctx_len,
    const float* __restrict__ cand, float* __restrict__ scores, int Hi, int max_pages, int page_size, int num_pages,
    int stride, int tiles_per_wave, int chunks_per_row) {
  const int b = blockIdx.x / chunks_per_row;
  const int chunk = blockIdx.x - b * chunks_per_row;
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;  // key column of the tile / head row of the query operand
  const int h = lane >> 5;  // lane half: which 64 dims of the key this lane supplies

  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  const int t_begin = (chunk * IDX_WAVES + wave) * tiles_per_wave;
  const int t_end = min(t_begin + tiles_per_wave, tiles_row);
  if (t_begin >= t_end) return;
  int L = stride;
  if (ctx_len) L = min(max(ctx_len[b], 0), stride);

  // Query operand: head 32m + j, dims 64h + 8s .. +7 at step s (zero rows past Hi).
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int head = 32 * m + j;
    const uint4* qp = reinterpret_cast<const uint4*>(q + ((size_t)b * Hi + (head < Hi ? head : 0)) * IDX_D + 64 * h);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      uint4 v = head < Hi ? qp[s] : make_uint4(0, 0, 0, 0);
      qa[m][s] = as_bf16x8(v);
    }
  }
  // Head weights in the accumulator layout: register r of head tile m holds head 32m + 8(r/4) + 4h + r%4.
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int head = 32 * m + 8 * (r >> 2) + 4 * h + (r & 3);
      wr[m][r] = head < Hi ? w[(size_t)b * Hi + head] : 0.0f;
    }

  const int* trow = table + (size_t)b * max_pages;
  auto load_tile = [&](int t, KeyTile& kt) {
    const int t0 = t * IDX_TILE;
    if (t0 < L) {
      const int page = safe_page(trow[t0 / page_size], num_pages);
      const size_t slot = (size_t)page * page_size + (t0 % page_size) + j;
      const uint4* kp = reinterpret_cast<const uint4*>(kcache + slot * IDX_D + 64 * h);
      kt.v[0] = load_stream16(kp + 0);
      kt.v[1] = load_stream16(kp + 1);
      kt.v[2] = load_stream16(kp + 2);
      kt.v[3] = load_stream16(kp + 3);
      kt.scale = kscale[slot];
    }
  };

  float* srow = scores + (size_t)b * stride;
  const float* crow = cand ? cand + (size_t)b * stride : nullptr;
  KeyTile cur, nxt;
  load_tile(t_begin, cur);
  for (int t = t_begin; t < t_end; ++t) {
    if (t + 1 < t_end) load_tile(t + 1, nxt);
    const int t0 = t * IDX_TILE;
    const int pos = t0 + j;
    float v = NEG_INF;
    if (t0 < L) {
      f32x16 acc[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint4 kv = cur.v[s >> 1];
        const bf16x8 kb = (s & 1) ? fp8x8_to_bf16x8(kv.z, kv.w) : fp8x8_to_bf16x8(kv.x, kv.y);
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kb, acc[m], 0, 0, 0);
      }
      float part = 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], fmaxf(acc[m][r], 0.0f), part);
      part += __shfl_xor(part, 32, WAVE);
      v = part * cur.scale;
      if (crow && pos < stride) v += crow[pos];
      if (pos >= L) v = NEG_INF;
    }
    if (h == 0 && pos < stride) srow[pos] = v;
    cur = nxt;
  }
}

template <int MT>
static hipError_t launch_indexer_mt(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                    const int* table, const int* ctx_len, const float* cand, float* scores, int B,
                                    int Hi, int max_pages, int page_size, int num_pages, int stride,
                                    int tiles_per_wave, hipStream_t stream) {
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  const int waves_row = (tiles_row + tiles_per_wave - 1) / tiles_per_wave;
  const int chunks_row = (waves_row + IDX_WAVES - 1) / IDX_WAVES;
  hipLaunchKernelGGL(indexer_decode_kernel<MT>, dim3(B * chunks_row), dim3(IDX_THREADS), 0, stream, q, w, k, ks,
                     table, ctx_len, cand, scores, Hi, max_pages, page_size, num_pages, stride, tiles_per_wave,
                     chunks_row);
  return hipGetLastError();
}

hipError_t launch_indexer_decode(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                 const int* table, const int* ctx_len, const float* cand, float* scores, int B,
                                 int Hi, int max_pages, int page_size, int num_pages, int stride, int num_cu,
                                 hipStream_t stream) {
  // About 4 waves per CU over the whole batch, each with at least one and at most 64 tiles.
  const long tiles = (long)B * ((stride + IDX_TILE - 1) / IDX_TILE);
  const long waves = (long)num_cu * 4;
  int tpw = (int)((tiles + waves - 1) / waves);
  tpw = tpw < 1 ? 1 : (tpw > 64 ? 64 : tpw);
  if (Hi <= 32)
    return launch_indexer_mt<1>(q, w, k, ks, table, ctx_len, cand, scores, B, Hi, max_pages, page_size, num_pages,
                                stride, tpw, stream);
  return launch_indexer_mt<2>(q, w, k, ks, table, ctx_len, cand, scores, B, Hi, max_pages, page_size, num_pages,
                              stride, tpw, stream);
}

}  // namespace dsa
