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
constexpr int IDX_PF = 4;         // key tiles in flight per wave (a ring of register buffers)
constexpr int IDX_QROW = IDX_D + 8;  // LDS row stride of the staged queries (bf16 elements; padding spreads banks)
constexpr int IDX_HSHIFT = 20;       // the top-k kernel's first-level bins: the top 12 bits of the order key
constexpr int IDX_HBINS = 4096;

struct KeyTile {
  uint4 v[4];  // 64 key bytes of this lane
  float scale;
};

// MT: query-head tiles of 32 (Hi <= 32 MT). Each wave scores `tiles_per_wave` consecutive 32-key tiles of one row,
// keeping IDX_PF tiles' loads in flight: a tile's buffer is refilled with the tile IDX_PF ahead as soon as its MFMAs
// have consumed it. The row's queries and head weights are staged once per workgroup in LDS. HIST: also accumulate
// the row's first-level top-k histogram into hist.
template <int MT, bool HIST>
__global__ __launch_bounds__(IDX_THREADS, 2) void indexer_decode_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint8_t* __restrict__ kcache,
    const float* __restrict__ kscale, const int* __restrict__ table, const int* __restrict__ ctx_len,
    const float* __restrict__ cand, float* __restrict__ scores, int* __restrict__ hist, int Hi, int max_pages,
    int page_size, int num_pages, int stride, int tiles_per_wave, int chunks_per_row) {
  __shared__ uint16_t qs[32 * MT * IDX_QROW];
  __shared__ float ws[32 * MT];
  __shared__ int hs[HIST ? IDX_HBINS : 1];  // the workgroup's share of the row's top-k histogram
  const int b = blockIdx.x / chunks_per_row;
  const int chunk = blockIdx.x - b * chunks_per_row;
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;  // key column of the tile / head row of the query operand
  const int h = lane >> 5;  // lane half: which 64 dims of the key this lane supplies

  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  int L = stride;
  if (ctx_len) L = min(max(ctx_len[b], 0), stride);
  const int t_begin = (chunk * IDX_WAVES + wave) * tiles_per_wave;
  const int t_end = min(t_begin + tiles_per_wave, tiles_row);
  const int* trow = table + (size_t)b * max_pages;

  auto load_tile = [&](int t, KeyTile& kt) {
    const int t0 = t * IDX_TILE;
    if (t < t_end && t0 < L) {
      const int page = safe_page(trow[t0 / page_size], num_pages);
      const size_t slot = (size_t)page * page_size + (t0 % page_size) + j;
      const uint8_t* kp = kcache + slot * IDX_D + 64 * h;
      kt.v[0] = load_stream16(kp + 0);
      kt.v[1] = load_stream16(kp + 16);
      kt.v[2] = load_stream16(kp + 32);
      kt.v[3] = load_stream16(kp + 48);
      kt.scale = kscale[slot];
    }
  };
  // the first tiles' loads go out before the query staging
  KeyTile buf[IDX_PF];
#pragma unroll
  for (int i = 0; i < IDX_PF; ++i) load_tile(t_begin + i, buf[i]);

  // stage the row's queries (zero rows past Hi) and head weights
  for (int i = threadIdx.x; i < 32 * MT * (IDX_D / 8); i += IDX_THREADS) {
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (head < Hi) v = *reinterpret_cast<const uint4*>(q + ((size_t)b * Hi + head) * IDX_D + 8 * c);
    *reinterpret_cast<uint4*>(&qs[head * IDX_QROW + 8 * c]) = v;
  }
  for (int i = threadIdx.x; i < 32 * MT; i += IDX_THREADS) ws[i] = i < Hi ? w[(size_t)b * Hi + i] : 0.0f;
  if (HIST)
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) hs[i] = 0;
  __syncthreads();

  // query operand: head 32m + j, dims 64h + 8s .. +7 at step s
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qa[m][s] = as_bf16x8(*reinterpret_cast<const uint4*>(&qs[(32 * m + j) * IDX_QROW + 64 * h + 8 * s]));
  // head weights in the accumulator layout: register r of head tile m holds head 32m + 8(r/4) + 4h + r%4
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) wr[m][r] = ws[32 * m + 8 * (r >> 2) + 4 * h + (r & 3)];

  float* srow = scores + (size_t)b * stride;
  const float* crow = cand ? cand + (size_t)b * stride : nullptr;
  for (int tg = t_begin; tg < t_end; tg += IDX_PF) {  // empty for a wave past the row's tiles
#pragma unroll
    for (int i = 0; i < IDX_PF; ++i) {
      const int t = tg + i;
      if (t < t_end) {
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
            const uint4 kv = buf[i].v[s >> 1];
            const bf16x8 kb = (s & 1) ? fp8x8_to_bf16x8(kv.z, kv.w) : fp8x8_to_bf16x8(kv.x, kv.y);
#pragma unroll
            for (int m = 0; m < MT; ++m)
              acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kb, acc[m], 0, 0, 0);
          }
          const float ksc = buf[i].scale;
          load_tile(t + IDX_PF, buf[i]);  // the buffer's operands are in the MFMA pipeline: refill it
          float part = 0.0f;
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], fmaxf(acc[m][r], 0.0f), part);
          part += __shfl_xor(part, 32, WAVE);
          v = part * ksc;
          if (crow && pos < stride) v += crow[pos];
          if (pos >= L) v = NEG_INF;
        }
        if (h == 0 && pos < stride) {
          srow[pos] = v;
          if (HIST && v > VISIBLE) atomicAdd(&hs[order_key(v) >> IDX_HSHIFT], 1);
        }
      }
    }
  }
  if (HIST) {
    // the row's first-level top-k histogram (top 12 bits of the order key of the selectable scores)
    __syncthreads();
    int* hrow = hist + (size_t)b * IDX_HBINS;
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) {
      const int c = hs[i];
      if (c) atomicAdd(&hrow[i], c);
    }
  }
}

template <int MT>
static hipError_t launch_indexer_mt(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                    const int* table, const int* ctx_len, const float* cand, float* scores,
                                    int* hist, int B, int Hi, int max_pages, int page_size, int num_pages, int stride,
                                    int tiles_per_wave, hipStream_t stream) {
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  const int waves_row = (tiles_row + tiles_per_wave - 1) / tiles_per_wave;
  const int chunks_row = (waves_row + IDX_WAVES - 1) / IDX_WAVES;
  if (hist)
    launch("indexer_decode_kernel", (indexer_decode_kernel<MT, true>), dim3(B * chunks_row), dim3(IDX_THREADS), stream, q, w,
                       k, ks, table, ctx_len, cand, scores, hist, Hi, max_pages, page_size, num_pages, stride,
                       tiles_per_wave, chunks_row);
  else
    launch("indexer_decode_kernel", (indexer_decode_kernel<MT, false>), dim3(B * chunks_row), dim3(IDX_THREADS), stream, q, w,
                       k, ks, table, ctx_len, cand, scores, hist, Hi, max_pages, page_size, num_pages, stride,
                       tiles_per_wave, chunks_row);
  return hipGetLastError();
}

hipError_t launch_indexer_decode(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                 const int* table, const int* ctx_len, const float* cand, float* scores,
                                 int* hist, int B, int Hi, int max_pages, int page_size, int num_pages, int stride,
                                 int num_cu, hipStream_t stream) {
  // Two workgroups (8 waves) per CU over the whole batch; a wave takes a multiple of the prefetch depth in tiles.
  const long tiles = (long)B * ((stride + IDX_TILE - 1) / IDX_TILE);
  const long waves = (long)num_cu * 2 * IDX_WAVES;
  int tpw = (int)((tiles + waves - 1) / waves);
  tpw = (tpw + IDX_PF - 1) / IDX_PF * IDX_PF;
  tpw = tpw < IDX_PF ? IDX_PF : tpw;
  if (Hi <= 32)
    return launch_indexer_mt<1>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                                num_pages, stride, tpw, stream);
  return launch_indexer_mt<2>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                              num_pages, stride, tpw, stream);
}

}  // namespace dsa
