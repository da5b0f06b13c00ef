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
constexpr int IDX_TPW = 4;        // key tiles per wave, streamed IDX_AHEAD ahead of the compute
constexpr int IDX_TPG = IDX_TPW * IDX_WAVES;  // key tiles per workgroup
constexpr int IDX_QROW = IDX_D + 8;  // LDS row stride of the staged queries (bf16 elements; padding spreads banks)
constexpr int IDX_HSHIFT = 20;       // the top-k kernel's first-level bins: the top 12 bits of the order key
constexpr int IDX_HBINS = HIST_BINS;

__device__ __forceinline__ float crow_value(const float* cand, int b, int stride, int pos) {
  return cand[(size_t)b * stride + pos];
}

constexpr int IDX_AHEAD = 1;  // key tiles a wave has in flight ahead of the one it computes (1, 2 and 3 measured)

hipError_t launch_indexer_decode_long(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                      const int* table, const int* ctx_len, float* scores, float* bm, int sub_log2,
                                      int nb, int* hist, int B, int Hi, int max_pages, int page_size, int num_pages,
                                      int stride, int num_cu, hipStream_t s);

// One 32-key tile's loads for lane (key j, half h): 64 key bytes (dims 64h .. 64h + 63) and the key's scale (a tile
// past the context reads the null page: every load is unconditional, so the waits count exactly).
template <bool CAND>
__device__ __forceinline__ void indexer_tile_loads(const uint8_t* __restrict__ kcache, const float* __restrict__ kscale,
                                                   const float* __restrict__ cand, int page, int t0, int L, int b,
                                                   int stride, int page_size, int j, int h, u32x4 (&kv)[4],
                                                   float& ksc, float& kc) {
  const size_t slot = t0 < L ? (size_t)page * page_size + (t0 % page_size) + j : (size_t)j;
  const uint8_t* kp = kcache + slot * IDX_D + 64 * h;
#pragma unroll
  for (int c = 0; c < 4; ++c) kv[c] = *reinterpret_cast<const u32x4*>(kp + 16 * c);
  ksc = kscale[slot];
  if (CAND) kc = crow_value(cand, b, stride, t0 < L ? min(t0 + j, stride - 1) : 0);
}

// MT: query-head tiles of 32 (Hi <= 32 MT). Each wave scores IDX_TPW consecutive 32-key tiles of one row as
// straight-line code: it reads the tiles' page ids (one per lane), then streams the tiles: the first IDX_AHEAD
// tiles' key bytes and scales are loaded up front, and each later tile is issued once the tile IDX_AHEAD before it
// has arrived, just before that tile's MFMAs, so its load overlaps their compute. (All of a wave's tiles loaded at
// once made the data of most waves arrive together at the end of the launch's memory window, with the compute
// after it: 12.4 us at config 2 against 10.6 us streamed one tile ahead, 11.7 two ahead.) Every load is
// unconditional (a tile past the context reads the null page and its score is replaced by NEG_INF), which keeps
// the waits exact. The row's queries and head weights are staged once per workgroup in LDS, their loads issued
// before the key loads.
// HIST: also accumulate the row's first-level top-k histogram into hist. CAND: add cand to the scores.
template <int MT, bool HIST, bool CAND>
__global__ __launch_bounds__(IDX_THREADS, 2) void indexer_decode_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint8_t* __restrict__ kcache,
    const float* __restrict__ kscale, const int* __restrict__ table, const int* __restrict__ ctx_len,
    const float* __restrict__ cand, float* __restrict__ scores, int* __restrict__ hist, int Hi, int max_pages,
    int page_size, int num_pages, int stride, int groups_per_row) {
  __shared__ uint16_t qs[32 * MT * IDX_QROW];
  __shared__ float ws[32 * MT];
  __shared__ int hs[HIST ? IDX_HBINS : 1];  // the workgroup's share of the row's top-k histogram
  const int b = blockIdx.x / groups_per_row;
  const int grp = blockIdx.x - b * groups_per_row;
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;  // key column of the tile / head row of the query operand
  const int h = lane >> 5;  // lane half: which 64 dims of the key this lane supplies

  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  int L = stride;
  if (ctx_len) L = min(max(ctx_len[b], 0), stride);
  const int t_begin = grp * IDX_TPG + wave * IDX_TPW;
  const int* trow = table + (size_t)b * max_pages;
  float* srow = scores + (size_t)b * stride;

  // the queries' loads first (each thread's 16-byte pieces, kept in registers until the LDS write)
  constexpr int QPT = 32 * MT * (IDX_D / 8) / IDX_THREADS;  // 16-byte query pieces per thread
  uint4 qv[QPT];
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    qv[r] = *reinterpret_cast<const uint4*>(q + ((size_t)b * Hi + min(head, Hi - 1)) * IDX_D + 8 * c);
  }
  const float wv = w[(size_t)b * Hi + min((int)threadIdx.x, Hi - 1)];

  // lane i < IDX_TPW: the page of tile t_begin + i (0, the null page, past the context)
  int pages;
  {
    const int t = t_begin + min(lane, IDX_TPW - 1);
    const int pg = trow[min(t * IDX_TILE / page_size, max_pages - 1)];  // independent of L: issued with its load
    pages = t * IDX_TILE < L ? safe_page(pg, num_pages) : 0;
  }

  // a tile's loads: 64 key bytes per lane (key j, dims 64h .. 64h + 63) and the key's scale; the first IDX_AHEAD
  // tiles now, each later one once the tile IDX_AHEAD before it has arrived
  u32x4 kv[IDX_TPW][4];
  float ksc[IDX_TPW], kc[IDX_TPW];
#pragma unroll
  for (int i = 0; i < IDX_AHEAD; ++i)
    indexer_tile_loads<CAND>(kcache, kscale, cand, __shfl(pages, i, WAVE), (t_begin + i) * IDX_TILE, L, b, stride,
                             page_size, j, h, kv[i], ksc[i], kc[i]);

  // stage the row's queries (zero rows past Hi) and head weights
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    *reinterpret_cast<uint4*>(&qs[head * IDX_QROW + 8 * c]) = head < Hi ? qv[r] : make_uint4(0, 0, 0, 0);
  }
  if (threadIdx.x < 32 * MT) ws[threadIdx.x] = (int)threadIdx.x < Hi ? wv : 0.0f;
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

#pragma unroll
  for (int i = 0; i < IDX_TPW; ++i) {
    if (i + IDX_AHEAD < IDX_TPW) {
      // tile i has arrived (the tiles after it may still be in flight, and the previous tile's score store): issue
      // tile i + IDX_AHEAD, so the wave streams its tiles behind its compute instead of waiting for all of them (the
      // compiler's own wait before tile i's first use keeps the data exact whatever this count admits)
      constexpr int OPS = CAND ? 6 : 5;  // vector memory operations of one tile's loads
      constexpr int WAIT = vmcnt_wait(OPS * (IDX_AHEAD - 1) + 1);
      __builtin_amdgcn_s_waitcnt(WAIT);
      __builtin_amdgcn_sched_barrier(0);
      indexer_tile_loads<CAND>(kcache, kscale, cand, __shfl(pages, i + IDX_AHEAD, WAVE),
                               (t_begin + i + IDX_AHEAD) * IDX_TILE, L, b, stride, page_size, j, h, kv[i + IDX_AHEAD],
                               ksc[i + IDX_AHEAD], kc[i + IDX_AHEAD]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int t = t_begin + i;
    const int pos = t * IDX_TILE + j;
    f32x16 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 k4 = kv[i][s >> 1];
      const bf16x8 kb = (s & 1) ? fp8x8_to_bf16x8(k4[2], k4[3]) : fp8x8_to_bf16x8(k4[0], k4[1]);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kb, acc[m], 0, 0, 0);
    }
    float part = 0.0f;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], relu(acc[m][r]), part);
    part += __shfl_xor(part, 32, WAVE);
    float v = CAND ? part * ksc[i] + kc[i] : part * ksc[i];
    if (pos >= L) v = NEG_INF;
    if (t < tiles_row && h == 0 && pos < stride) {
      srow[pos] = v;
      if (HIST && v > VISIBLE) atomicAdd(&hs[order_key(v) >> IDX_HSHIFT], 1);
    }
  }
  if (HIST) {
    // the row's first-level top-k histogram (top 12 bits of the order key of the selectable scores)
    __syncthreads();
    int* hrow = hist + ((size_t)b * HIST_REPLICAS + grp % HIST_REPLICAS) * IDX_HBINS;
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) {
      const int c = hs[i];
      if (c) atomicAdd(&hrow[i], c);
    }
  }
}

// Long rows (the separate kernels' indexer past 32,768 tokens): the same wave layout and arithmetic, but each wave
// streams up to 64 consecutive tiles of one row through a ring of IL_AHEAD + 1 register tiles, IL_AHEAD in flight
// ahead of the one it computes, so the row's queries are staged once per workgroup for up to 8,192 keys instead of 512
// and the memory stream runs without the workgroups' start-up gaps. The wave's page ids are one load per lane (tile
// tw0 + lane). HIST: also the row's top-k first-level histogram (as the kernel above). BM: also the two-level top-k's
// first-level sub-block maxima, bm[b, p / sub] = the maximum of the scores of positions p .. p + sub - 1 (sub a power
// of two up to 32: a tile's 32 keys hold whole sub-blocks), for p < nb sub.
//
// Work split (TW = 0, rows' lengths given, B <= 256): the grid's workgroups share the batch's live tiles (those
// holding a position below the row's length) evenly, whatever the rows' lengths: every workgroup reads the B
// lengths, and with T live tiles in all and G workgroups, each wave takes cw = ceil(T / (4 (G - B))) consecutive
// tiles of one row, row b taking ceil(T_b / 4 cw) workgroups (at most G in all); the tiles past each row's length
// (NEG_INF scores and maxima) are shared out the same way, ceil(Q / G) of the Q of them a workgroup. (A fixed TW
// tiles a wave: row b takes wgs_per_row workgroups whatever its length, those past it writing NEG_INF.)
constexpr int IL_AHEAD = 2;
constexpr int IL_RING = IL_AHEAD + 1;
constexpr int IL_TW_MAX = 64;
constexpr int IL_BAL_MAXB = IDX_THREADS;  // rows of a batch the even split takes (one a thread)

// Exclusive prefix sum over the workgroup's IDX_THREADS threads (one value each) and the total; sc holds
// IDX_WAVES + 1 ints (written, then read after a barrier; the caller's next use of sc waits for a barrier of its own).
__device__ __forceinline__ int il_block_excl(int v, int* sc, int* total) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  const int inc = wave_incl_scan(v);
  if (lane == WAVE - 1) sc[wave] = inc;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w2 = 0; w2 < IDX_WAVES; ++w2) {
    const int t = sc[w2];
    before += w2 < wave ? t : 0;
    all += t;
  }
  *total = all;
  return before + inc - v;
}

template <int MT, bool BM, bool HIST>
__global__ __launch_bounds__(IDX_THREADS, 2) void indexer_decode_long_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint8_t* __restrict__ kcache,
    const float* __restrict__ kscale, const int* __restrict__ table, const int* __restrict__ ctx_len,
    float* __restrict__ scores, float* __restrict__ bm, int sub_log2, int nb, int* __restrict__ hist, int Hi,
    int max_pages, int page_size, int num_pages, int stride, int TW, int wgs_per_row, int B) {
  __shared__ uint16_t qs[32 * MT * IDX_QROW];
  __shared__ float ws[32 * MT];
  __shared__ int hs[HIST ? IDX_HBINS : 1];  // the workgroup's share of the row's top-k histogram
  // the even split: each row's first tail tile in the batch's tail order, its live tiles; the scan's scratch; the
  // workgroup's row (-1: none) and its first tile
  __shared__ int bal[2 * IL_BAL_MAXB + IDX_WAVES + 2];
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31, h = lane >> 5;
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  int b, L, tw0, n_t, n_live;
  if (TW == 0) {  // (launch-uniform) the even split of the live tiles
    const int t = threadIdx.x, G = gridDim.x, g = blockIdx.x;
    int* sc = bal + 2 * IL_BAL_MAXB;
    int* wrow = sc + IDX_WAVES;
    if (t == 0) wrow[0] = -1;
    const int Lt = t < B ? min(max(ctx_len[t], 0), stride) : 0;
    const int Tt = min((Lt + IDX_TILE - 1) / IDX_TILE, tiles_row);  // row t's live tiles
    int T, Q, wgs;
    il_block_excl(Tt, sc, &T);
    const int cw = max((T + 4 * (G - B) - 1) / (4 * (G - B)), 1);  // tiles a wave (at most 64: the launch's G)
    const int mt = (Tt + 4 * cw - 1) / (4 * cw);                   // row t's workgroups
    __syncthreads();  // sc read by every thread
    const int Mt = il_block_excl(mt, sc, &wgs);
    if (t < B && g >= Mt && g < Mt + mt) {
      wrow[0] = t;
      wrow[1] = (g - Mt) * 4 * cw;  // the workgroup's first tile of the row
    }
    const int Pt = t < B ? tiles_row - Tt : 0;  // row t's tiles past its length
    __syncthreads();  // sc read by every thread
    const int Ut = il_block_excl(Pt, sc, &Q);
    if (t < B) {
      bal[t] = Ut;
      bal[IL_BAL_MAXB + t] = Tt;
    }
    __syncthreads();
    // the tiles past the rows' lengths, tail tile u of ceil(Q / G) a workgroup: 8 tiles a pass, 32 lanes a tile
    const int qg = (Q + G - 1) / G, u0 = g * qg, u1 = min(u0 + qg, Q);
    for (int u = u0 + t / IDX_TILE; u < u1; u += IDX_THREADS / IDX_TILE) {
      int lo = 0, hi = B - 1;  // the last row whose tail starts at or before u
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (bal[mid] <= u) lo = mid; else hi = mid - 1;
      }
      const int tile = bal[IL_BAL_MAXB + lo] + (u - bal[lo]);
      const int pos = tile * IDX_TILE + (t & (IDX_TILE - 1));
      if (pos < stride) scores[(size_t)lo * stride + pos] = NEG_INF;
      if (BM) {
        if (sub_log2 == 5) {
          if ((t & (IDX_TILE - 1)) == 0 && tile < nb) bm[(size_t)lo * nb + tile] = NEG_INF;
        } else if ((pos & ((1 << sub_log2) - 1)) == 0 && (pos >> sub_log2) < nb) {
          bm[(size_t)lo * nb + (pos >> sub_log2)] = NEG_INF;
        }
      }
    }
    b = wrow[0];
    if (b < 0) return;  // (workgroup-uniform) a workgroup past the rows' shares
    L = min(max(ctx_len[b], 0), stride);
    tw0 = wrow[1] + wave * cw;
    n_live = n_t = max(min(cw, bal[IL_BAL_MAXB + b] - tw0), 0);
  } else {
    b = blockIdx.x / wgs_per_row;
    const int grp = blockIdx.x - b * wgs_per_row;
    L = ctx_len ? min(max(ctx_len[b], 0), stride) : stride;
    tw0 = (grp * IDX_WAVES + wave) * TW;                                // this wave's first tile
    n_t = max(min(TW, tiles_row - tw0), 0);                             // its tiles in the row
    n_live = max(min(n_t, (L + IDX_TILE - 1) / IDX_TILE - tw0), 0);  // those with keys of the context
  }
  float* srow = scores + (size_t)b * stride;

  constexpr int QPT = 32 * MT * (IDX_D / 8) / IDX_THREADS;
  uint4 qv[QPT];
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    qv[r] = *reinterpret_cast<const uint4*>(q + ((size_t)b * Hi + min(head, Hi - 1)) * IDX_D + 8 * c);
  }
  const float wv = w[(size_t)b * Hi + min((int)threadIdx.x, Hi - 1)];
  int pages;  // lane i: the page of tile tw0 + i (0, the null page, past the context)
  {
    const int t = tw0 + lane;
    const int pg = table[(size_t)b * max_pages + min(t * IDX_TILE / page_size, max_pages - 1)];
    pages = t * IDX_TILE < L ? safe_page(pg, num_pages) : 0;
  }
  u32x4 kv[IL_RING][4];
  float ksc[IL_RING], kc_unused;
#pragma unroll
  for (int r = 0; r < IL_AHEAD; ++r)
    indexer_tile_loads<false>(kcache, kscale, nullptr, __shfl(pages, r, WAVE), (tw0 + r) * IDX_TILE, L, b, stride,
                              page_size, j, h, kv[r], ksc[r], kc_unused);
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    *reinterpret_cast<uint4*>(&qs[head * IDX_QROW + 8 * c]) = head < Hi ? qv[r] : make_uint4(0, 0, 0, 0);
  }
  if (threadIdx.x < 32 * MT) ws[threadIdx.x] = (int)threadIdx.x < Hi ? wv : 0.0f;
  if (HIST)
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) hs[i] = 0;
  __syncthreads();
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qa[m][s] = as_bf16x8(*reinterpret_cast<const uint4*>(&qs[(32 * m + j) * IDX_QROW + 64 * h + 8 * s]));
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) wr[m][r] = ws[32 * m + 8 * (r >> 2) + 4 * h + (r & 3)];
  const int sub = 1 << sub_log2;
  int tmr = __float_as_int(NEG_INF);  // tiles of 32 (sub_log2 = 5): lane i holds the maximum of the wave's tile i

  for (int i0 = 0; i0 < n_live; i0 += IL_RING) {
#pragma unroll
    for (int r = 0; r < IL_RING; ++r) {
      const int i = i0 + r;  // ring slot r
      if (i >= n_live) break;  // wave-uniform
      // tile i has arrived (the IL_AHEAD - 1 tiles after it and the last tiles' stores may still be out): issue tile
      // i + IL_AHEAD into the slot tile i - 1 left (a tile past the wave's range reads its keys, unused); the
      // compiler's own wait before tile i's first use keeps the data exact whatever this count admits
      // (stores a tile: the score, and with sub-blocks below 32 their maxima)
      if (BM && sub_log2 < 5)
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(5 * (IL_AHEAD - 1) + 2 * IL_AHEAD));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(5 * (IL_AHEAD - 1) + IL_AHEAD));
      __builtin_amdgcn_sched_barrier(0);
      {
        const int ia = i + IL_AHEAD;
        const int pa = ia < IL_TW_MAX ? __shfl(pages, ia, WAVE) : 0;
        indexer_tile_loads<false>(kcache, kscale, nullptr, pa, (tw0 + ia) * IDX_TILE, L, b, stride, page_size, j,
                                  h, kv[(r + IL_AHEAD) % IL_RING], ksc[(r + IL_AHEAD) % IL_RING], kc_unused);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int pos = (tw0 + i) * IDX_TILE + j;
      f32x16 acc[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int x = 0; x < 16; ++x) acc[m][x] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const u32x4 k4 = kv[r][s >> 1];
        const bf16x8 kb = (s & 1) ? fp8x8_to_bf16x8(k4[2], k4[3]) : fp8x8_to_bf16x8(k4[0], k4[1]);
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kb, acc[m], 0, 0, 0);
      }
      float part = 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int x = 0; x < 16; ++x) part = fmaf(wr[m][x], relu(acc[m][x]), part);
      part += __shfl_xor(part, 32, WAVE);
      const float v = pos < L ? part * ksc[r] : NEG_INF;
      if (h == 0 && pos < stride) {
        srow[pos] = v;
        if (HIST && v > VISIBLE) atomicAdd(&hs[order_key(v) >> IDX_HSHIFT], 1);
      }
      if (BM) {
        if (sub_log2 == 5) {
          // (uniform) the tile's maximum by DPP (each row of 16 lanes, then row 0's into row 1) into lane i of tmr
          float mx = row_max(v);
          mx = fmaxf(mx, __int_as_float(dpp<0x142, 0xa, false>(__float_as_int(mx))));
          const int m16 = __builtin_amdgcn_readlane(__float_as_int(mx), 16);
          tmr = lane == i ? m16 : tmr;
        } else {
          float mx = v;
          for (int d = 1; d < sub; d <<= 1) mx = max_nonan(mx, __shfl_xor(mx, d, WAVE));
          if (h == 0 && (j & (sub - 1)) == 0 && (pos >> sub_log2) < nb) bm[(size_t)b * nb + (pos >> sub_log2)] = mx;
        }
      }
    }
  }
  // the wave's tiles past the context: NEG_INF (and their sub-block maxima)
  for (int e = lane; e < (n_t - n_live) * IDX_TILE; e += WAVE) {
    const int pos = (tw0 + n_live) * IDX_TILE + e;
    if (pos < stride) srow[pos] = NEG_INF;
    if (BM && sub_log2 < 5 && (pos & ((1 << sub_log2) - 1)) == 0 && (pos >> sub_log2) < nb)
      bm[(size_t)b * nb + (pos >> sub_log2)] = NEG_INF;
  }
  // tiles of 32: the wave's tile maxima in one store (NEG_INF past the context)
  if (BM && sub_log2 == 5 && lane < n_t && tw0 + lane < nb) bm[(size_t)b * nb + tw0 + lane] = __int_as_float(tmr);
  if (HIST) {
    // the row's first-level top-k histogram (top 12 bits of the order key of the selectable scores)
    __syncthreads();
    int* hrow = hist + (size_t)b * HIST_REPLICAS * IDX_HBINS;
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) {
      const int c = hs[i];
      if (c) atomicAdd(&hrow[i], c);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the loads of the tiles past the range have landed before the wave ends
}

template <int MT, bool BM, bool HIST>
static hipError_t launch_indexer_long_v(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                        const int* table, const int* ctx_len, float* scores, float* bm, int sub_log2,
                                        int nb, int* hist, int B, int Hi, int max_pages, int page_size, int num_pages,
                                        int stride, int num_cu, hipStream_t s) {
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  if (ctx_len && B <= IL_BAL_MAXB) {
    // the even split: two workgroups per CU (four per CU, or three tiles in flight instead of two, measured slower at
    // configs 3 and 4), more when the batch's tiles need them at 64 a wave
    const long need = B + ((long)B * tiles_row + IDX_WAVES * IL_TW_MAX - 1) / (IDX_WAVES * IL_TW_MAX);
    const long G = need > 2L * num_cu ? need : 2L * num_cu;
    return launch("indexer_decode_long_kernel", indexer_decode_long_kernel<MT, BM, HIST>, dim3((unsigned)G),
                  dim3(IDX_THREADS), s, q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, hist, Hi, max_pages,
                  page_size, num_pages, stride, 0, 0, B);
  }
  // tiles per wave: about two workgroups per CU over the batch at its longest rows, 4 to 64 tiles each
  const long waves_target = 2L * num_cu * IDX_WAVES;
  int TW = (int)(((long)B * tiles_row + waves_target - 1) / waves_target);
  TW = TW < 4 ? 4 : (TW > IL_TW_MAX ? IL_TW_MAX : TW);
  const int wgs_row = (tiles_row + IDX_WAVES * TW - 1) / (IDX_WAVES * TW);
  return launch("indexer_decode_long_kernel", indexer_decode_long_kernel<MT, BM, HIST>, dim3(B * wgs_row),
                dim3(IDX_THREADS), s, q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, hist, Hi, max_pages,
                page_size, num_pages, stride, TW, wgs_row, B);
}

template <int MT>
static hipError_t launch_indexer_long_mt(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                         const int* table, const int* ctx_len, float* scores, float* bm, int sub_log2,
                                         int nb, int* hist, int B, int Hi, int max_pages, int page_size,
                                         int num_pages, int stride, int num_cu, hipStream_t s) {
  if (hist && bm)
    return launch_indexer_long_v<MT, true, true>(q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, hist, B, Hi,
                                                 max_pages, page_size, num_pages, stride, num_cu, s);
  if (hist)
    return launch_indexer_long_v<MT, false, true>(q, w, k, ks, table, ctx_len, scores, nullptr, 0, 0, hist, B, Hi,
                                                  max_pages, page_size, num_pages, stride, num_cu, s);
  if (bm)
    return launch_indexer_long_v<MT, true, false>(q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, nullptr, B,
                                                  Hi, max_pages, page_size, num_pages, stride, num_cu, s);
  return launch_indexer_long_v<MT, false, false>(q, w, k, ks, table, ctx_len, scores, nullptr, 0, 0, nullptr, B, Hi,
                                                 max_pages, page_size, num_pages, stride, num_cu, s);
}

// The long-row indexer (no additive candidates): with the top-k's first-level histogram accumulated into hist
// [B, 4096] when given, and with sub-block maxima bm [B, nb] when bm is given (1 << sub_log2 <= 32): the two-level
// selection's first level, or (with the histogram) the maxima of the 32-key tiles that the long rows' one-launch
// selection reads instead of the scores.
hipError_t launch_indexer_decode_long(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                      const int* table, const int* ctx_len, float* scores, float* bm, int sub_log2,
                                      int nb, int* hist, int B, int Hi, int max_pages, int page_size, int num_pages,
                                      int stride, int num_cu, hipStream_t s) {
  if (bm && (sub_log2 < 1 || sub_log2 > 5)) return hipErrorInvalidValue;
  if (Hi <= 32)
    return launch_indexer_long_mt<1>(q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, hist, B, Hi, max_pages,
                                     page_size, num_pages, stride, num_cu, s);
  return launch_indexer_long_mt<2>(q, w, k, ks, table, ctx_len, scores, bm, sub_log2, nb, hist, B, Hi, max_pages,
                                   page_size, num_pages, stride, num_cu, s);
}

template <int MT, bool HIST, bool CAND>
static hipError_t launch_indexer_variant(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                         const int* table, const int* ctx_len, const float* cand, float* scores,
                                         int* hist, int B, int Hi, int max_pages, int page_size, int num_pages,
                                         int stride, hipStream_t stream) {
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  const int groups_row = (tiles_row + IDX_TPG - 1) / IDX_TPG;
  return launch("indexer_decode_kernel", indexer_decode_kernel<MT, HIST, CAND>, dim3(B * groups_row),
                dim3(IDX_THREADS), stream, q, w, k, ks, table, ctx_len, cand, scores, hist, Hi, max_pages, page_size,
                num_pages, stride, groups_row);
}

template <int MT>
static hipError_t launch_indexer_mt(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                    const int* table, const int* ctx_len, const float* cand, float* scores,
                                    int* hist, int B, int Hi, int max_pages, int page_size, int num_pages, int stride,
                                    hipStream_t s) {
  if (hist && cand)
    return launch_indexer_variant<MT, true, true>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages,
                                                  page_size, num_pages, stride, s);
  if (hist)
    return launch_indexer_variant<MT, true, false>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi,
                                                   max_pages, page_size, num_pages, stride, s);
  if (cand)
    return launch_indexer_variant<MT, false, true>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi,
                                                   max_pages, page_size, num_pages, stride, s);
  return launch_indexer_variant<MT, false, false>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages,
                                                  page_size, num_pages, stride, s);
}

hipError_t launch_indexer_decode(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                 const int* table, const int* ctx_len, const float* cand, float* scores,
                                 int* hist, int B, int Hi, int max_pages, int page_size, int num_pages, int stride,
                                 int num_cu, hipStream_t stream) {
  if (!hist && !cand && stride > 32 * 1024)  // long rows: the streaming form
    return launch_indexer_decode_long(q, w, k, ks, table, ctx_len, scores, nullptr, 0, 0, nullptr, B, Hi, max_pages,
                                      page_size, num_pages, stride, num_cu, stream);
  if (Hi <= 32)
    return launch_indexer_mt<1>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                                num_pages, stride, stream);
  return launch_indexer_mt<2>(q, w, k, ks, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                              num_pages, stride, stream);
}

// The pooled indexer's form (trnrt/kernels/dsa_index.py:243-268 `scores` over GLM's pool-key cache,
// trnrt/models/mla.py:628-629): bf16 keys with no per-key scale, pages of any power-of-two number of keys (a page of
// 64 tokens holds 16 pools of kpool 4):
//
//   score[b, p] = sum_h w[b, h] * relu(q[b, h, :] . k_bf16[slot(b, p), :])   (+ cand[b, p]),  NEG_INF at p >= L_b
//
// Same wave layout as above (lane (j, h): key j of the tile, dims 64h .. 64h + 63, here 128 bytes of bf16 fed to
// the MFMA as they are), but every lane looks up its own key's page, so a 32-key tile may span pages: one round of
// page-id loads, then one round of key loads, as above. A key is 256 bytes here against 132 there, so a wave takes
// BF_TPW tiles (half as many): the same bytes in flight per lane and twice the workgroups over a row.
constexpr int BF_TPW = 2;
constexpr int BF_TPG = BF_TPW * IDX_WAVES;

template <int MT, bool HIST, bool CAND>
__global__ __launch_bounds__(IDX_THREADS, 2) void indexer_decode_bf16_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const uint16_t* __restrict__ kcache,
    const int* __restrict__ table, const int* __restrict__ ctx_len, const float* __restrict__ cand,
    float* __restrict__ scores, int* __restrict__ hist, int Hi, int max_pages, int page_size, int num_pages,
    int stride, int groups_per_row) {
  __shared__ uint16_t qs[32 * MT * IDX_QROW];
  __shared__ float ws[32 * MT];
  __shared__ int hs[HIST ? IDX_HBINS : 1];  // the workgroup's share of the row's top-k histogram
  const int b = blockIdx.x / groups_per_row;
  const int grp = blockIdx.x - b * groups_per_row;
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;
  const int h = lane >> 5;
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  int L = stride;
  if (ctx_len) L = min(max(ctx_len[b], 0), stride);
  const int t_begin = grp * BF_TPG + wave * BF_TPW;
  const int* trow = table + (size_t)b * max_pages;
  float* srow = scores + (size_t)b * stride;

  constexpr int QPT = 32 * MT * (IDX_D / 8) / IDX_THREADS;
  uint4 qv[QPT];
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    qv[r] = *reinterpret_cast<const uint4*>(q + ((size_t)b * Hi + min(head, Hi - 1)) * IDX_D + 8 * c);
  }
  const float wv = w[(size_t)b * Hi + min((int)threadIdx.x, Hi - 1)];

  // this lane's key in each of its tiles: its page (the null page past the context), then its 128 bytes
  int page[BF_TPW];
#pragma unroll
  for (int i = 0; i < BF_TPW; ++i) {
    const int p = (t_begin + i) * IDX_TILE + j;
    const int pg = trow[min(p / page_size, max_pages - 1)];
    page[i] = p < L ? safe_page(pg, num_pages) : 0;
  }
  // the first tile's keys now, each later one once the one before it has arrived (as in the FP8 form)
  u32x4 kv[BF_TPW][8];
  float kc[BF_TPW];
  auto tile_loads = [&](int i, u32x4(&kvi)[8], float& kci) __attribute__((always_inline)) {
    const int p = (t_begin + i) * IDX_TILE + j;
    const size_t slot = (size_t)page[i] * page_size + (p < L ? p % page_size : 0);
    const uint16_t* kp = kcache + slot * IDX_D + 64 * h;
#pragma unroll
    for (int c = 0; c < 8; ++c) kvi[c] = *reinterpret_cast<const u32x4*>(kp + 8 * c);
    if (CAND) kci = crow_value(cand, b, stride, p < L ? min(p, stride - 1) : 0);
  };
  tile_loads(0, kv[0], kc[0]);

#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = threadIdx.x + r * IDX_THREADS;
    const int head = i / (IDX_D / 8), c = i - head * (IDX_D / 8);
    *reinterpret_cast<uint4*>(&qs[head * IDX_QROW + 8 * c]) = head < Hi ? qv[r] : make_uint4(0, 0, 0, 0);
  }
  if (threadIdx.x < 32 * MT) ws[threadIdx.x] = (int)threadIdx.x < Hi ? wv : 0.0f;
  if (HIST)
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) hs[i] = 0;
  __syncthreads();
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qa[m][s] = as_bf16x8(*reinterpret_cast<const uint4*>(&qs[(32 * m + j) * IDX_QROW + 64 * h + 8 * s]));
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) wr[m][r] = ws[32 * m + 8 * (r >> 2) + 4 * h + (r & 3)];

#pragma unroll
  for (int i = 0; i < BF_TPW; ++i) {
    if (i + 1 < BF_TPW) {
      constexpr int WAIT = vmcnt_wait(1);  // tile i in (the previous tile's score store may be in flight)
      __builtin_amdgcn_s_waitcnt(WAIT);
      __builtin_amdgcn_sched_barrier(0);
      tile_loads(i + 1, kv[i + 1], kc[i + 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int t = t_begin + i;
    const int pos = t * IDX_TILE + j;
    f32x16 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], __builtin_bit_cast(bf16x8, kv[i][s]), acc[m], 0, 0,
                                                         0);
    float part = 0.0f;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], relu(acc[m][r]), part);
    part += __shfl_xor(part, 32, WAVE);
    float v = CAND ? part + kc[i] : part;
    if (pos >= L) v = NEG_INF;
    if (t < tiles_row && h == 0 && pos < stride) {
      srow[pos] = v;
      if (HIST && v > VISIBLE) atomicAdd(&hs[order_key(v) >> IDX_HSHIFT], 1);
    }
  }
  if (HIST) {
    __syncthreads();
    int* hrow = hist + ((size_t)b * HIST_REPLICAS + grp % HIST_REPLICAS) * IDX_HBINS;
    for (int i = threadIdx.x; i < IDX_HBINS; i += IDX_THREADS) {
      const int c = hs[i];
      if (c) atomicAdd(&hrow[i], c);
    }
  }
}

template <int MT, bool HIST, bool CAND>
static hipError_t launch_indexer_bf16_variant(const uint16_t* q, const float* w, const uint16_t* k, const int* table,
                                              const int* ctx_len, const float* cand, float* scores, int* hist, int B,
                                              int Hi, int max_pages, int page_size, int num_pages, int stride,
                                              hipStream_t stream) {
  const int tiles_row = (stride + IDX_TILE - 1) / IDX_TILE;
  const int groups_row = (tiles_row + BF_TPG - 1) / BF_TPG;
  return launch("indexer_decode_bf16_kernel", indexer_decode_bf16_kernel<MT, HIST, CAND>, dim3(B * groups_row),
                dim3(IDX_THREADS), stream, q, w, k, table, ctx_len, cand, scores, hist, Hi, max_pages, page_size,
                num_pages, stride, groups_row);
}

template <int MT>
static hipError_t launch_indexer_bf16_mt(const uint16_t* q, const float* w, const uint16_t* k, const int* table,
                                         const int* ctx_len, const float* cand, float* scores, int* hist, int B,
                                         int Hi, int max_pages, int page_size, int num_pages, int stride,
                                         hipStream_t s) {
  if (hist && cand)
    return launch_indexer_bf16_variant<MT, true, true>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi, max_pages,
                                                       page_size, num_pages, stride, s);
  if (hist)
    return launch_indexer_bf16_variant<MT, true, false>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi,
                                                        max_pages, page_size, num_pages, stride, s);
  if (cand)
    return launch_indexer_bf16_variant<MT, false, true>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi,
                                                        max_pages, page_size, num_pages, stride, s);
  return launch_indexer_bf16_variant<MT, false, false>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi, max_pages,
                                                       page_size, num_pages, stride, s);
}

// hist (or null): the rows' first-level top-k histograms, accumulated (the workspace region the top-k reads with
// hist_ready; zero on entry).
hipError_t launch_indexer_decode_bf16(const uint16_t* q, const float* w, const uint16_t* k, const int* table,
                                      const int* ctx_len, const float* cand, float* scores, int* hist, int B, int Hi,
                                      int max_pages, int page_size, int num_pages, int stride, hipStream_t s) {
  if (Hi <= 32)
    return launch_indexer_bf16_mt<1>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                                     num_pages, stride, s);
  return launch_indexer_bf16_mt<2>(q, w, k, table, ctx_len, cand, scores, hist, B, Hi, max_pages, page_size,
                                   num_pages, stride, s);
}

}  // namespace dsa
