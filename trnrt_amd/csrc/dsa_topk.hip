// Exact per-row top-k for gfx950 (the selection rule of trnrt/models/dsa_select.py:10-38 and
// trnrt/kernels/dsa_topk.py:10-40, output form of trnrt/models/dsa_long.py:94-112 `_ascending`):
// per row, the `keep` largest selectable scores; every selected score >= every unselected one; among the scores
// equal to the keep-th largest, the lowest positions; only scores > VISIBLE are selectable (vis_only); a row with
// fewer selectable scores than keep selects all of them. Output: the positions in ascending order plus the count.
//
// One workgroup of 1024 threads owns a row of up to 32,768 scores, held in registers as order-preserving integer
// keys (dsa_common.h order_key), so every comparison is exact (the reference's radix search over the threshold's bit
// pattern, dsa_topk.py:19-26, is exact for the same reason). The threshold T (the keep-th largest key) is found
// radix-wise from the top: a histogram of the top 12 key bits (accumulated by the indexer while it writes the
// scores, or built here in LDS), then LDS histograms of the next 11 and the last 9 bits over the keys that share the
// prefix found so far, each pass a block-wide suffix scan for the bin holding the need-th key. The selection is
// every key > T plus the first `room` keys equal to T by position, written in position order by a block-wide prefix
// count, so no list is sorted and no key moves.
//
// Longer rows go through the reference's two-level exact selection (trnrt/models/dsa_long.py:26-42, 114-132):
// sub-block maxima, the top-keep sub-blocks, and the top-keep of their elements in position order.
#include "dsa_common.h"

namespace dsa {

constexpr int TK_HSHIFT = 20;  // first level: the top 12 bits of the order key
constexpr int TK_HBINS = HIST_BINS;
constexpr int TR_THREADS = 1024;
constexpr int TR_WAVES = TR_THREADS / WAVE;
constexpr int TR_MAXG = 8;     // float4 groups per thread: rows of up to 4 x 8 x 1024 scores

// The row length in elements of a selection level: len[row] for a flat row; ceil(len / len_div) for sub-block
// maxima; len[row] * len_mul for a candidate row of len[row] sub-blocks; at most stride.
__device__ __forceinline__ int level_len(const int* len, int row, int len_div, int len_mul, int stride) {
  if (!len) return stride;
  long l = len[row];
  l = l < 0 ? 0 : l;
  if (len_div > 1) l = (l + len_div - 1) / len_div;
  if (len_mul > 1) l *= len_mul;
  return (int)(l < stride ? l : stride);
}

// Branch-free (masks, not selects), so that the compiler keeps the loads feeding it unconditional.
__device__ __forceinline__ uint32_t select_key(float v, int vis_only) {
  return order_key(v) & (0u - (uint32_t)(!vis_only || v > VISIBLE));
}

// Four keys of positions p .. p + 3 of a row of `stride` scores (0 past L or not selectable), loaded
// unconditionally from in-range addresses so that the waits on the loads count exactly: VEC (stride a multiple of
// 4, at least 4) one float4, clamped to the row's last four (a clamped p is past the row, so all four are masked);
// otherwise four scalar loads clamped to the row.
template <bool VEC>
__device__ __forceinline__ void load_keys4(const float* srow, int stride, int L, int p, int vis_only, uint32_t (&k)[4]) {
  float v[4];
  if (VEC) {
    const float4 f = *reinterpret_cast<const float4*>(srow + min(p, stride - 4));
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = srow[min(p + c, stride - 1)];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) k[c] = select_key(v[c], vis_only) & (0u - (uint32_t)(p + c < L));
}

// Sum over the 16 lanes of each DPP row (quad swaps, then the half-row and row mirrors), in every lane of the row.
__device__ __forceinline__ int row16_sum(int v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}

// Optional second output of a flat selection: the cache slot of each selected position through the row's page table
// (slot = page_table[row, p / page_size] * page_size + p % page_size, pages clamped into the cache), and for the
// entries past the count the slot of position 0, the slot the attention reads for them.
struct SlotOut {
  const int* table;
  int max_pages, page_size, num_pages;
  int* rows;  // [B, keep], or null
};

// p / page_size and p % page_size of a position p >= 0: shifts when the page size is a power of two (page_shift >= 0),
// which keeps the integer division out of the per-key output loops.
__device__ __forceinline__ int page_of(int p, int ps, int page_shift) {
  return page_shift >= 0 ? p >> page_shift : p / ps;
}
__device__ __forceinline__ int page_shift_of(int ps) { return (ps & (ps - 1)) ? -1 : __builtin_ctz((unsigned)ps); }

// The second level of a two-level selection read in place (the row kernel's IND form): candidate position p of a
// row is score src(p) = bidx[row, p / sub] sub + p % sub of the original row (sub a multiple of 4, so a float4 of
// candidates is one float4 of scores), live while p / sub < bcnt[row] and src < len[row]; the selection is written
// in the reference's form: pools int64 (the src positions) and vals (their scores), NEG_INF / 0 past the count, cnt
// int64.
struct IndOut {
  const float* scores;
  int stride;
  const int* len;
  const int* bidx;
  const int* bcnt;
  int sub;
  int64_t* pools;
  int64_t* cnt;
  float* vals;
};

struct RowShared {
  int pg[TR_THREADS];               // page ids of the row's first 1024 pages (slot output)
  int bins[TK_HBINS];               // the current pass's histogram (4096, 2048 or 512 bins in key order)
  int wtot[TR_WAVES];               // per-wave totals of a block scan
  uint32_t blk[TR_MAXG * TR_WAVES];  // output: per (group, wave) packed counts, then their exclusive prefix
  int sel_bin, sel_above;
};

// Block-wide, over sh.bins[0 .. nbins) (a key histogram, higher bins = larger keys): the bin holding the need-th
// largest key (*bin) and the keys in the bins above it (*above); returns the total count. Each thread takes
// nbins / 1024 bins (at least one; threads past nbins take none). sh.sel_bin must be -1 on entry (set before the
// barrier that precedes the histogram's atomics); counts that cannot hold the need-th key give bin 0, above 0. The
// caller must pass a barrier before sh.sel_bin / sh.wtot are written again.
__device__ int row_find_bin(RowShared& sh, int nbins, int need, int* bin, int* above) {
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int per = nbins >= TR_THREADS ? nbins / TR_THREADS : 1;
  const int first = t * per;
  int hb[4];
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[i] = (i < per && first + i < nbins) ? sh.bins[first + i] : 0;
    mine += hb[i];
  }
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;  // inclusive suffix over the lanes
  if (lane == 0) sh.wtot[wave] = inc;
  __syncthreads();
  int after = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < TR_WAVES; ++w) {
    const int x = sh.wtot[w];
    after += w > wave ? x : 0;
    tot += x;
  }
  int excl = after + inc - mine;  // keys in the bins above this thread's
  if (excl < need && excl + mine >= need) {
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      if (i < per && first + i < nbins && excl < need) {
        if (excl + hb[i] >= need) {
          sh.sel_bin = first + i;
          sh.sel_above = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int b = sh.sel_bin;
  *bin = b < 0 ? 0 : b;
  *above = b < 0 ? 0 : sh.sel_above;
  return tot;
}

// The flat selection: one workgroup per row (blockIdx.x) of up to 4 G 1024 scores. Thread t holds the keys of
// positions 4 (1024 e + t) + c, e < G, c < 4 (coalesced float4 loads). HIST_IN: the row's top-12-bit histogram is in
// hist[row] (read, then zeroed for the next call); otherwise it is built here.
// IND: the row is the IndOut second level (scores / stride / len are unused; stride is the candidate row length).
template <int G, bool HIST_IN, bool VEC, bool ROWS, bool IND = false, bool OUT64 = false>
__global__ __launch_bounds__(TR_THREADS) void topk_row_kernel(const float* __restrict__ scores, int stride,
                                                              const int* __restrict__ len, int len_div, int len_mul,
                                                              int keep, int vis_only, int* __restrict__ hist,
                                                              int* __restrict__ idx_out, int* __restrict__ cnt_out,
                                                              SlotOut so, IndOut io) {
  __shared__ RowShared sh;
  const int row = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = IND ? stride : level_len(len, row, len_div, len_mul, stride);
  const float* srow = scores + (size_t)row * stride;

  int4 h4r[HIST_REPLICAS];
  int* hrow = hist + (size_t)row * HIST_REPLICAS * TK_HBINS;
  if (HIST_IN)
#pragma unroll
    for (int r = 0; r < HIST_REPLICAS; ++r) h4r[r] = reinterpret_cast<const int4*>(hrow + r * TK_HBINS)[t];
  int pgv = 0;
  if (ROWS) pgv = so.table[(size_t)row * so.max_pages + min(t, so.max_pages - 1)];
  uint32_t key[G][4];
  int src[G];  // IND: the original position of each float4 group's first candidate
  if (IND) {
    const int nblk = min(io.bcnt[row], keep);
    const int Lo = min(max(io.len[row], 0), io.stride);
    int bsrc[G];
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const int p = 4 * (TR_THREADS * e + t);
      const int k = min(p / io.sub, keep - 1);
      bsrc[e] = io.bidx[(size_t)row * keep + k];
    }
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const int p = 4 * (TR_THREADS * e + t);
      const int k = p / io.sub;
      const bool blive = p < stride && k < nblk;
      src[e] = blive ? bsrc[e] * io.sub + (p - k * io.sub) : 0;  // live positions are below Lo <= io.stride
      const float4 f =
          *reinterpret_cast<const float4*>(io.scores + (size_t)row * io.stride + min(max(src[e], 0), io.stride - 4));
      const float v[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) key[e][c] = select_key(v[c], vis_only) & (0u - (uint32_t)(blive && src[e] + c < Lo));
    }
  } else {
#pragma unroll
    for (int e = 0; e < G; ++e) load_keys4<VEC>(srow, stride, L, 4 * (TR_THREADS * e + t), vis_only, key[e]);
  }
  if (ROWS) sh.pg[t] = safe_page(pgv, so.num_pages);
  if (t == 0) sh.sel_bin = -1;
  if (HIST_IN) {
    int4 h4 = h4r[0];
#pragma unroll
    for (int r = 1; r < HIST_REPLICAS; ++r) {
      h4.x += h4r[r].x;
      h4.y += h4r[r].y;
      h4.z += h4r[r].z;
      h4.w += h4r[r].w;
    }
    reinterpret_cast<int4*>(sh.bins)[t] = h4;
#pragma unroll
    for (int r = 0; r < HIST_REPLICAS; ++r)
      reinterpret_cast<int4*>(hrow + r * TK_HBINS)[t] = make_int4(0, 0, 0, 0);  // zero for the next call
    __syncthreads();
  } else {
    reinterpret_cast<int4*>(sh.bins)[t] = make_int4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[e][c]) atomicAdd(&sh.bins[key[e][c] >> TK_HSHIFT], 1);
    __syncthreads();
  }

  // the threshold, 12 + 11 + 9 bits
  int c0, above;
  const int nvis = row_find_bin(sh, TK_HBINS, keep, &c0, &above);
  uint32_t T = 0;
  int room = 0;
  if (nvis > keep) {
    int need = keep - above;
    __syncthreads();  // every thread has read the pass's result
    reinterpret_cast<int2*>(sh.bins)[t] = make_int2(0, 0);
    if (t == 0) sh.sel_bin = -1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[e][c] && (key[e][c] >> TK_HSHIFT) == (uint32_t)c0) atomicAdd(&sh.bins[(key[e][c] >> 9) & 2047], 1);
    __syncthreads();
    int c1;
    row_find_bin(sh, 2048, need, &c1, &above);
    need -= above;
    const uint32_t pre = ((uint32_t)c0 << 11) | (uint32_t)c1;  // the top 23 bits of T
    __syncthreads();
    if (t < 512) sh.bins[t] = 0;
    if (t == 0) sh.sel_bin = -1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[e][c] && (key[e][c] >> 9) == pre) atomicAdd(&sh.bins[key[e][c] & 511], 1);
    __syncthreads();
    int c2;
    row_find_bin(sh, 512, need, &c2, &above);
    T = (pre << 9) | (uint32_t)c2;
    room = need - above;  // keys equal to T to take, lowest positions first
    room = room < 0 ? 0 : room;
  }

  // per (group, wave): keys above T and keys equal to T, packed hi / lo 16 bits (each at most 32768)
  uint32_t mine[G], incl[G];
#pragma unroll
  for (int e = 0; e < G; ++e) {
    uint32_t na = 0, nt = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      na += key[e][c] > T;
      nt += T != 0 && key[e][c] == T;
    }
    mine[e] = (na << 16) | nt;
    incl[e] = wave_incl_scan_u32(mine[e]);
    if (lane == WAVE - 1) sh.blk[e * TR_WAVES + wave] = incl[e];
  }
  __syncthreads();
  if (wave == 0) {  // exclusive prefix over (group, wave) in position order: G x 16 <= 128 values, 2 per lane
    const uint32_t x0 = 2 * lane < G * TR_WAVES ? sh.blk[2 * lane] : 0u;
    const uint32_t x1 = 2 * lane + 1 < G * TR_WAVES ? sh.blk[2 * lane + 1] : 0u;
    const uint32_t in2 = wave_incl_scan_u32(x0 + x1);
    const uint32_t ex = in2 - x0 - x1;
    if (2 * lane < G * TR_WAVES) sh.blk[2 * lane] = ex;
    if (2 * lane + 1 < G * TR_WAVES) sh.blk[2 * lane + 1] = ex + x0;
  }
  __syncthreads();
  int* orow = idx_out + (size_t)row * keep;
  const int psh = ROWS ? page_shift_of(so.page_size) : 0;
#pragma unroll
  for (int e = 0; e < G; ++e) {
    const uint32_t before = sh.blk[e * TR_WAVES + wave] + incl[e] - mine[e];
    int a_before = (int)(before >> 16), t_before = (int)(before & 0xffffu);
    const int p0 = 4 * (TR_THREADS * e + t);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool a = key[e][c] > T;
      const bool ti = T != 0 && key[e][c] == T;
      const bool sel = a || (ti && t_before < room);
      const int o = a_before + (t_before < room ? t_before : room);
      if (sel && (unsigned)o < (unsigned)keep) {  // in range whatever the counts
        if (IND || OUT64) {  // the reference's outputs: int64 positions, their scores
          io.pools[(size_t)row * keep + o] = (IND ? src[e] : p0) + c;
          io.vals[(size_t)row * keep + o] = key_to_float(key[e][c]);
        } else {
          orow[o] = p0 + c;
        }
        if (ROWS) {
          const int ps = so.page_size, pi = page_of(p0 + c, ps, psh);
          so.rows[(size_t)row * keep + o] = sh.pg[min(pi, TR_THREADS - 1)] * ps + (p0 + c - pi * ps);
        }
      }
      a_before += a;
      t_before += ti;
    }
  }
  const int cnt_row = nvis < keep ? nvis : keep;
  for (int i = cnt_row + t; i < keep; i += TR_THREADS) {
    if (IND || OUT64) {
      io.pools[(size_t)row * keep + i] = 0;
      io.vals[(size_t)row * keep + i] = NEG_INF;
    } else {
      orow[i] = 0;
    }
    if (ROWS) so.rows[(size_t)row * keep + i] = sh.pg[0] * so.page_size;
  }
  if (t == 0) {
    if (IND || OUT64)
      io.cnt[row] = cnt_row;
    else
      cnt_out[row] = cnt_row;
  }
}

// The chunked selection of rows of more than 4096 scores: workgroups of 256 threads own chunks of 2048 positions
// (thread t the positions base + 4 (256 e + t) + c, e < 2, c < 4), so the per-key work is spread over many CUs, in
// two kernels with one round of global loads each:
//   topk_chunk_kernel:  from the row's top-12-bit histogram the threshold's bin c0 and the keys in bins above it
//                       (every chunk computes them); per chunk the count of its keys above c0 and its keys in bin
//                       c0 (the candidates, a few hundred per row for indexer scores), written in position order;
//   topk_output_kernel: every chunk loads the row's candidates and counts, finds T and the ties to take with two LDS
//                       histogram passes (bits 19..9, then 8..0), each chunk's output base from the per-chunk counts,
//                       and writes its own selected positions in order.
constexpr int TC_THREADS = 256;
constexpr int TC_WAVES = TC_THREADS / WAVE;
constexpr int TC_CHUNK = 2048;
constexpr int TC_MAXCH = 16;   // rows of up to 32,768 scores
constexpr int TC_CAND = 128;   // candidates per chunk held in registers by the output kernel (more: extra rounds)
constexpr int TKH_THREADS = 256;  // histogram kernel: 8 scores per thread, 2048 per workgroup

struct RowMeta {
  int c0;      // the threshold's 12-bit bin, -1 when the row has at most keep selectable keys
  int above0;  // selectable keys in bins above c0
  int nvis;    // selectable keys of the row
  int pad;
  int n_a[TC_MAXCH];  // per chunk: keys above c0 (all its selectable keys when c0 is -1)
  int n_c[TC_MAXCH];  // per chunk: keys in bin c0
};

// The first level of a standalone selection: the histogram of the top 12 bits of the selectable keys of each row,
// accumulated into hist[row, 4096] (zero before; the output kernel zeroes it again). 2048 scores per workgroup.
__global__ __launch_bounds__(TKH_THREADS) void topk_hist_kernel(const float* __restrict__ scores, int stride,
                                                                const int* __restrict__ len, int len_div,
                                                                int len_mul, int vis_only, int* __restrict__ hist) {
  __shared__ int h[TK_HBINS];
  const int row = blockIdx.y;
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = blockIdx.x * TC_CHUNK;
  if (base >= L) return;  // the whole workgroup: no barrier is skipped by part of it
  for (int i = threadIdx.x; i < TK_HBINS; i += TKH_THREADS) h[i] = 0;
  __syncthreads();
  const float* srow = scores + (size_t)row * stride;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int p = base + e * TKH_THREADS + threadIdx.x;
    if (p < L) {
      const uint32_t k = select_key(srow[p], vis_only);
      if (k) atomicAdd(&h[k >> TK_HSHIFT], 1);
    }
  }
  __syncthreads();
  int* hrow = hist + ((size_t)row * HIST_REPLICAS + blockIdx.x % HIST_REPLICAS) * TK_HBINS;
  for (int i = threadIdx.x; i < TK_HBINS; i += TKH_THREADS) {
    const int c = h[i];
    if (c) atomicAdd(&hrow[i], c);
  }
}

// A chunk's 8 keys per thread.
template <bool VEC>
__device__ __forceinline__ void load_chunk_keys(const float* srow, int stride, int L, int base, int vis_only,
                                                uint32_t (&key)[2][4]) {
#pragma unroll
  for (int e = 0; e < 2; ++e) load_keys4<VEC>(srow, stride, L, base + 4 * (TC_THREADS * e + (int)threadIdx.x), vis_only, key[e]);
}

// Exclusive prefix, in position order (group e, then wave, then lane), of per-thread packed counts mine[e]
// (hi / lo 16 bits, block totals below 65536); blk: 2 x TC_WAVES words of LDS. Two barriers.
__device__ __forceinline__ void chunk_prefix(const uint32_t (&mine)[2], uint32_t* blk, uint32_t (&before)[2]) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  uint32_t incl[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    incl[e] = wave_incl_scan_u32(mine[e]);
    if (lane == WAVE - 1) blk[e * TC_WAVES + wave] = incl[e];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t acc = 0;
    const int me = e * TC_WAVES + wave;
#pragma unroll
    for (int i = 0; i < 2 * TC_WAVES; ++i) acc += i < me ? blk[i] : 0u;
    before[e] = acc + incl[e] - mine[e];
  }
  __syncthreads();
}

struct ChunkShared {
  int wtot[TC_WAVES];
  uint32_t blk[2 * TC_WAVES];
  int c0, above0;
};

template <bool VEC>
__global__ __launch_bounds__(TC_THREADS) void topk_chunk_kernel(const float* __restrict__ scores, int stride,
                                                                const int* __restrict__ len, int len_div,
                                                                int len_mul, int keep, int vis_only,
                                                                const int* __restrict__ hist,
                                                                RowMeta* __restrict__ meta,
                                                                uint32_t* __restrict__ ckey) {
  __shared__ ChunkShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = chunk * TC_CHUNK;
  // one round of loads: the thread's 16 histogram bins and its 8 keys
  const int4* h4 = reinterpret_cast<const int4*>(hist + (size_t)row * HIST_REPLICAS * TK_HBINS) + 4 * t;
  int4 hv[4 * HIST_REPLICAS];
#pragma unroll
  for (int i = 0; i < 4 * HIST_REPLICAS; ++i) hv[i] = h4[(i / 4) * (TK_HBINS / 4) + i % 4];
  uint32_t key[2][4];
  load_chunk_keys<VEC>(scores + (size_t)row * stride, stride, L, base, vis_only, key);
  int hb[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[4 * i] = hv[i].x;
    hb[4 * i + 1] = hv[i].y;
    hb[4 * i + 2] = hv[i].z;
    hb[4 * i + 3] = hv[i].w;
  }
#pragma unroll
  for (int r = 1; r < HIST_REPLICAS; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hb[4 * i] += hv[4 * r + i].x;
      hb[4 * i + 1] += hv[4 * r + i].y;
      hb[4 * i + 2] += hv[4 * r + i].z;
      hb[4 * i + 3] += hv[4 * r + i].w;
    }
  // c0: the bin holding the keep-th largest key (bins 16t .. 16t + 15 on thread t; suffix over threads)
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) mine += hb[i];
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;  // inclusive suffix over the lanes
  if (lane == 0) sh.wtot[wave] = inc;
  if (t == 0) {
    sh.c0 = -1;
    sh.above0 = 0;
  }
  __syncthreads();
  int after = 0, nvis = 0;
#pragma unroll
  for (int w = 0; w < TC_WAVES; ++w) {
    const int x = sh.wtot[w];
    after += w > wave ? x : 0;
    nvis += x;
  }
  int excl = after + inc - mine;
  if (nvis > keep && excl < keep && excl + mine >= keep) {
#pragma unroll
    for (int i = 15; i >= 0; --i) {
      if (excl < keep) {
        if (excl + hb[i] >= keep) {
          sh.c0 = 16 * t + i;
          sh.above0 = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int c0 = sh.c0;
  // classify the chunk's keys: above c0 (all selectable ones when c0 is -1) and in bin c0 (the candidates)
  uint32_t mc[2];
  int na = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t nc = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = key[e][c];
      const int bin = (int)(k >> TK_HSHIFT);
      na += k != 0u && bin > c0;
      nc += k != 0u && bin == c0;
    }
    mc[e] = nc;
  }
  // position-ordered compaction of the candidates
  uint32_t before[2];
  chunk_prefix(mc, sh.blk, before);
  uint32_t* crow = ckey + ((size_t)row * TC_MAXCH + chunk) * TC_CHUNK;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t o = before[e];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = key[e][c];
      if (k != 0u && (int)(k >> TK_HSHIFT) == c0) {
        if (o < (uint32_t)TC_CHUNK) crow[o] = k;
        ++o;
      }
    }
  }
  // chunk totals: candidates = prefix of the last (e, wave) block + its count; above = block sum of na
  const int na_w = wave_sum(na);
  if (lane == 0) sh.wtot[wave] = na_w;
  __syncthreads();
  if (t == TC_THREADS - 1) {
    int na_tot = 0;
#pragma unroll
    for (int w = 0; w < TC_WAVES; ++w) na_tot += sh.wtot[w];
    const int nc_tot = (int)(before[1] + mc[1]);  // the last thread's exclusive prefix of e = 1 plus its own
    meta[row].n_a[chunk] = na_tot;
    meta[row].n_c[chunk] = nc_tot;
    if (chunk == 0) {
      meta[row].c0 = c0;
      meta[row].above0 = sh.above0;
      meta[row].nvis = nvis;
    }
  }
}

struct OutShared {
  int pg[WAVE];  // page ids of the chunk's positions (slot output; pages of at least 32 positions)
  int pg0;                    // the page of position 0
  int bins[2048];  // the 11-bit pass's histogram
  int bins2[512];  // the 9-bit pass's, zeroed with the first so the passes need no barrier between them
  int wtot[TC_WAVES];
  uint32_t blk[2 * TC_WAVES];
  int gt[TC_MAXCH], tie[TC_MAXCH], na[TC_MAXCH];
  int sel[2], sel2[2];  // each pass's result: the bin, the keys above it
};

// Block-wide (256 threads) over bins[0 .. nbins) (nbins 2048 or 512, higher bins = larger keys): the bin holding the
// need-th largest key and the keys in the bins above it, through sel[0 .. 1]. sel[0] must be -1 on entry (written
// before the barrier preceding the histogram's atomics); inconsistent counts give bin 0, above 0. Two barriers.
__device__ void out_find_bin(OutShared& sh, const int* bins, int* sel, int nbins, int need, int* bin,
                             int* above) {
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int per = nbins / TC_THREADS;  // 8 or 2
  int hb[8];
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    hb[i] = i < per ? bins[per * t + i] : 0;
    mine += hb[i];
  }
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;  // inclusive suffix over the lanes
  if (lane == 0) sh.wtot[wave] = inc;
  __syncthreads();
  int after = 0;
#pragma unroll
  for (int w = 0; w < TC_WAVES; ++w) after += w > wave ? sh.wtot[w] : 0;
  int excl = after + inc - mine;
  if (excl < need && excl + mine >= need) {
#pragma unroll
    for (int i = 7; i >= 0; --i) {
      if (i < per && excl < need) {
        if (excl + hb[i] >= need) {
          sel[0] = per * t + i;
          sel[1] = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int b = sel[0];
  *bin = b < 0 ? 0 : b;
  *above = b < 0 ? 0 : sel[1];
}

template <bool VEC, bool ROWS>
__global__ __launch_bounds__(TC_THREADS) void topk_output_kernel(const float* __restrict__ scores, int stride,
                                                                 const int* __restrict__ len, int len_div,
                                                                 int len_mul, int keep, int vis_only, int nchunks,
                                                                 int* __restrict__ hist,
                                                                 const RowMeta* __restrict__ meta,
                                                                 const uint32_t* __restrict__ ckey,
                                                                 int* __restrict__ idx_out, int* __restrict__ cnt_out,
                                                                 SlotOut so) {
  __shared__ OutShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = chunk * TC_CHUNK;
  const int g = t >> 4, sub = t & 15;  // candidate group: chunk g, entries sub + 16 k
  // one round of loads: the row's meta, the first TC_CAND candidates of every chunk, the chunk's own keys
  const RowMeta& rm = meta[row];
  const int c0 = rm.c0, above0 = rm.above0, nvis = rm.nvis;
  const int l16 = lane & 15;
  int na_l = rm.n_a[l16], nc_l = rm.n_c[l16];
  const int live = 0 - (int)(l16 < nchunks);  // masks, not selects: the loads stay unconditional
  na_l = min(max(na_l, 0), TC_CHUNK) & live;
  nc_l = min(max(nc_l, 0), TC_CHUNK) & live;
  const uint32_t* cg = ckey + ((size_t)row * TC_MAXCH + g) * TC_CHUNK;
  uint32_t ck[TC_CAND / 16];
#pragma unroll
  for (int k = 0; k < TC_CAND / 16; ++k) ck[k] = cg[sub + 16 * k];
  const int pg_first = ROWS ? base / so.page_size : 0;
  int pgv = 0, pg0v = 0;
  if (ROWS) {
    pgv = so.table[(size_t)row * so.max_pages + min(pg_first + lane, so.max_pages - 1)];
    pg0v = so.table[(size_t)row * so.max_pages];
  }
  uint32_t key[2][4];
  load_chunk_keys<VEC>(scores + (size_t)row * stride, stride, L, base, vis_only, key);
  if (ROWS && wave == 0) {
    sh.pg[lane] = safe_page(pgv, so.num_pages);
    if (lane == 0) sh.pg0 = safe_page(pg0v, so.num_pages);
  }
  // leave the row's histogram zero for the next call (every topk_chunk_kernel workgroup has read it)
  int* hrow = hist + (size_t)row * HIST_REPLICAS * TK_HBINS;
  for (int i = chunk * TC_THREADS + t; i < HIST_REPLICAS * TK_HBINS; i += nchunks * TC_THREADS) hrow[i] = 0;

  const int ncg = __shfl(nc_l, g, WAVE);  // this thread's candidate chunk's count (lane g < 16 holds it)
  if (t < TC_MAXCH) sh.na[t] = na_l;
  const int maxc = (int)wave_max_u32((uint32_t)nc_l);
  uint32_t T = 0;
  int room = 0;
  if (c0 >= 0 && nvis > keep) {
    int need = keep - above0;
    // pass A: bits 19 .. 9 of the candidates (all in bin c0); pass B's bins and the per-chunk counts are cleared here
    // too
    for (int i = t; i < 2048; i += TC_THREADS) sh.bins[i] = 0;
    for (int i = t; i < 512; i += TC_THREADS) sh.bins2[i] = 0;
    if (t == 0) {
      sh.sel[0] = -1;
      sh.sel2[0] = -1;
    }
    if (t < TC_MAXCH) {
      sh.gt[t] = 0;
      sh.tie[t] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TC_CAND / 16; ++k)
      if (g < nchunks && sub + 16 * k < ncg) atomicAdd(&sh.bins[(ck[k] >> 9) & 2047], 1);
    for (int r = 1; r * TC_CAND < maxc; ++r)  // rare: chunks with more than TC_CAND candidates
      for (int k = 0; k < TC_CAND / 16; ++k) {
        const int i = r * TC_CAND + sub + 16 * k;
        if (g < nchunks && i < ncg) atomicAdd(&sh.bins[(cg[i] >> 9) & 2047], 1);
      }
    __syncthreads();
    int c1, above;
    out_find_bin(sh, sh.bins, sh.sel, 2048, need, &c1, &above);
    need -= above;
    const uint32_t pre = ((uint32_t)c0 << 11) | (uint32_t)c1;
    // pass B: bits 8 .. 0 of the candidates under the 23-bit prefix
#pragma unroll
    for (int k = 0; k < TC_CAND / 16; ++k)
      if (g < nchunks && sub + 16 * k < ncg && (ck[k] >> 9) == pre) atomicAdd(&sh.bins2[ck[k] & 511], 1);
    for (int r = 1; r * TC_CAND < maxc; ++r)
      for (int k = 0; k < TC_CAND / 16; ++k) {
        const int i = r * TC_CAND + sub + 16 * k;
        if (g < nchunks && i < ncg && (cg[i] >> 9) == pre) atomicAdd(&sh.bins2[cg[i] & 511], 1);
      }
    __syncthreads();
    int c2;
    out_find_bin(sh, sh.bins2, sh.sel2, 512, need, &c2, &above);
    T = (pre << 9) | (uint32_t)c2;
    room = need - above;
    room = room < 0 ? 0 : room;
    // per chunk: candidates above T and equal to T (a 16-lane group per chunk)
    int gtc = 0, tic = 0;
#pragma unroll
    for (int k = 0; k < TC_CAND / 16; ++k)
      if (sub + 16 * k < ncg) {
        gtc += ck[k] > T;
        tic += ck[k] == T;
      }
    for (int r = 1; r * TC_CAND < maxc; ++r)
      for (int k = 0; k < TC_CAND / 16; ++k) {
        const int i = r * TC_CAND + sub + 16 * k;
        if (i < ncg) {
          gtc += cg[i] > T;
          tic += cg[i] == T;
        }
      }
    gtc = row16_sum(gtc);  // the 16 lanes of a candidate group are one DPP row
    tic = row16_sum(tic);
    if (sub == 0 && g < nchunks) {
      sh.gt[g] = gtc;
      sh.tie[g] = tic;
    }
  } else if (t < TC_MAXCH) {
    sh.gt[t] = 0;
    sh.tie[t] = 0;
  }
  __syncthreads();
  // this chunk's output base and the ties it may take
  int out_base = 0, ties_before = 0;
  for (int j = 0; j < chunk && j < nchunks; ++j) {
    const int tj = sh.tie[j];
    int take = room - ties_before;
    take = take < 0 ? 0 : (take > tj ? tj : take);
    out_base += sh.na[j] + sh.gt[j] + take;
    ties_before += tj;
  }
  int room_here = room - ties_before;
  room_here = room_here < 0 ? 0 : room_here;

  // ordered output of the chunk: keys above T, and the first room_here keys equal to T
  uint32_t mine[2], before[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t na = 0, nt = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      na += key[e][c] > T;
      nt += T != 0u && key[e][c] == T;
    }
    mine[e] = (na << 16) | nt;
  }
  chunk_prefix(mine, sh.blk, before);
  int* orow = idx_out + (size_t)row * keep;
  const int psh = ROWS ? page_shift_of(so.page_size) : 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    int a_before = (int)(before[e] >> 16), t_before = (int)(before[e] & 0xffffu);
    const int p0 = base + 4 * (TC_THREADS * e + t);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool a = key[e][c] > T;
      const bool ti = T != 0u && key[e][c] == T;
      const bool sel = a || (ti && t_before < room_here);
      const int o = out_base + a_before + (t_before < room_here ? t_before : room_here);
      if (sel && (unsigned)o < (unsigned)keep) {  // in range whatever the counts
        orow[o] = p0 + c;
        if (ROWS) {
          const int ps = so.page_size, p = p0 + c, pi = page_of(p, ps, psh);
          so.rows[(size_t)row * keep + o] = sh.pg[min(pi - pg_first, WAVE - 1)] * ps + (p - pi * ps);
        }
      }
      a_before += a;
      t_before += ti;
    }
  }
  if (chunk == 0) {
    const int cnt_row = nvis < 0 ? 0 : (nvis < keep ? nvis : keep);
    for (int i = cnt_row + t; i < keep; i += TC_THREADS) {
      orow[i] = 0;
      if (ROWS) so.rows[(size_t)row * keep + i] = sh.pg0 * so.page_size;
    }
    if (t == 0) cnt_out[row] = cnt_row;
  }
}

// Rows longer than 32,768 scores in few rows (a decode batch at long context): the chunked selection above with any
// number of chunks, in three kernels over the row's first-level histogram (built by the indexer or topk_hist_kernel):
//   topk_long_chunk_kernel:   per chunk of 2,048 positions, the threshold's bin c0 from the histogram, the count of
//                             the chunk's keys above c0, and its keys in bin c0 (the candidates) in position order;
//   topk_long_resolve_kernel: one workgroup per row reads every chunk's candidates, finds T (the keep-th largest key)
//                             by two LDS histogram passes over their low 20 bits (11 + 9) and the ties to take, and
//                             gives each chunk its first output index and its ties taken (ties go to the lowest
//                             positions: chunk order, then position order inside a chunk);
//   topk_long_output_kernel:  every chunk writes its selected positions in order (and their cache slots).
// Candidates are held per chunk (at most its 2,048 keys), so the workspace bounds them whatever the scores.
constexpr int TL_MAXCH = 1024;  // chunks per row: rows of up to 2,097,152 scores
constexpr int TL_THREADS = 1024;
constexpr int TL_WAVES = TL_THREADS / WAVE;

struct LongRow {
  int c0, above0, nvis;  // as RowMeta
  uint32_t T;            // the threshold key (0: every selectable key is taken)
};

// Per-chunk arrays of the long selection, [B][nch] each, and the candidates [B][nch][TC_CHUNK].
struct LongBuffers {
  LongRow* row;
  int *na, *nc, *base, *take;
  uint32_t* cand;
};

template <bool VEC>
__global__ __launch_bounds__(TC_THREADS) void topk_long_chunk_kernel(const float* __restrict__ scores, int stride,
                                                                     const int* __restrict__ len, int keep,
                                                                     int vis_only, const int* __restrict__ hist,
                                                                     LongBuffers lb, int nch) {
  __shared__ ChunkShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = level_len(len, row, 1, 1, stride);
  const int base = chunk * TC_CHUNK;
  const int4* h4 = reinterpret_cast<const int4*>(hist + (size_t)row * HIST_REPLICAS * TK_HBINS) + 4 * t;
  int4 hv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) hv[i] = h4[i];
  uint32_t key[2][4];
  load_chunk_keys<VEC>(scores + (size_t)row * stride, stride, L, base, vis_only, key);
  int hb[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[4 * i] = hv[i].x;
    hb[4 * i + 1] = hv[i].y;
    hb[4 * i + 2] = hv[i].z;
    hb[4 * i + 3] = hv[i].w;
  }
  // c0: the bin holding the keep-th largest key (bins 16t .. 16t + 15 on thread t; suffix over threads)
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) mine += hb[i];
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;
  if (lane == 0) sh.wtot[wave] = inc;
  if (t == 0) {
    sh.c0 = -1;
    sh.above0 = 0;
  }
  __syncthreads();
  int after = 0, nvis = 0;
#pragma unroll
  for (int w = 0; w < TC_WAVES; ++w) {
    const int x = sh.wtot[w];
    after += w > wave ? x : 0;
    nvis += x;
  }
  int excl = after + inc - mine;
  if (nvis > keep && excl < keep && excl + mine >= keep) {
#pragma unroll
    for (int i = 15; i >= 0; --i) {
      if (excl < keep) {
        if (excl + hb[i] >= keep) {
          sh.c0 = 16 * t + i;
          sh.above0 = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int c0 = sh.c0;
  uint32_t mc[2];
  int na = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t nc = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = key[e][c];
      const int bin = (int)(k >> TK_HSHIFT);
      na += k != 0u && bin > c0;
      nc += k != 0u && bin == c0;
    }
    mc[e] = nc;
  }
  uint32_t before[2];
  chunk_prefix(mc, sh.blk, before);
  const size_t ci = (size_t)row * nch + chunk;
  uint32_t* crow = lb.cand + ci * TC_CHUNK;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t o = before[e];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = key[e][c];
      if (k != 0u && (int)(k >> TK_HSHIFT) == c0) {
        if (o < (uint32_t)TC_CHUNK) crow[o] = k;
        ++o;
      }
    }
  }
  const int na_w = wave_sum(na);
  if (lane == 0) sh.wtot[wave] = na_w;
  __syncthreads();
  if (t == TC_THREADS - 1) {
    int na_tot = 0;
#pragma unroll
    for (int w = 0; w < TC_WAVES; ++w) na_tot += sh.wtot[w];
    lb.na[ci] = na_tot;
    lb.nc[ci] = (int)(before[1] + mc[1]);
    if (chunk == 0) {
      lb.row[row].c0 = c0;
      lb.row[row].above0 = sh.above0;
      lb.row[row].nvis = nvis;
    }
  }
}

constexpr int TL_CAP = 4096;  // candidates of a row staged in LDS (more: read from the workspace)

struct LongShared {
  int bins[2048];
  int bins2[512];
  int gt[TL_MAXCH], tie[TL_MAXCH];
  int coff[TL_MAXCH];   // per chunk: its candidates' first flat index
  uint32_t sk[TL_CAP];  // the row's candidates in flat order (chunk order, then position order)
  uint16_t sj[TL_CAP];  // their chunks
  int wtot[TL_WAVES];
  int sel[2], sel2[2];
};

// Block-wide (1024 threads) over bins[0 .. nbins) (2048 or 512, higher bins = larger keys): the bin holding the
// need-th largest key and the keys above it through sel[0 .. 1] (sel[0] -1 on entry, written before a barrier that
// precedes this call). Two barriers; the caller passes one more before sel or wtot are written again.
__device__ void long_find_bin(LongShared& sh, const int* bins, int* sel, int nbins, int need, int* bin, int* above) {
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int per = nbins / TL_THREADS;  // 2, or 0 for 512 bins (thread t < 512 then takes bin t)
  int hb[2];
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int b = per ? per * t + i : (i == 0 ? t : nbins);
    hb[i] = b < nbins ? bins[b] : 0;
    mine += hb[i];
  }
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;
  if (lane == 0) sh.wtot[wave] = inc;
  __syncthreads();
  int after = 0;
#pragma unroll
  for (int w = 0; w < TL_WAVES; ++w) after += w > wave ? sh.wtot[w] : 0;
  int excl = after + inc - mine;
  if (excl < need && excl + mine >= need) {
#pragma unroll
    for (int i = 1; i >= 0; --i) {
      const int b = per ? per * t + i : (i == 0 ? t : nbins);
      if (b < nbins && excl < need) {
        if (excl + hb[i] >= need) {
          sel[0] = b;
          sel[1] = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int b = sel[0];
  *bin = b < 0 ? 0 : b;
  *above = b < 0 ? 0 : sel[1];
}

// Block-wide inclusive scan over the 1024 threads (thread order); the total into *tot. Two barriers.
__device__ __forceinline__ int long_block_scan(int v, int* wtot, int* tot) {
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int incl = wave_incl_scan(v);
  if (lane == WAVE - 1) wtot[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < TL_WAVES; ++w) {
    const int x = wtot[w];
    before += w < wave ? x : 0;
    all += x;
  }
  *tot = all;
  __syncthreads();
  return before + incl;
}

// The chunk of flat candidate index i (the last chunk whose first index is at most i; chunks without candidates
// share their successor's first index, so the search lands on the one holding i).
__device__ __forceinline__ int long_chunk_of(const int* coff, int nch, int i) {
  int lo = 0, hi = nch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (coff[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(TL_THREADS) void topk_long_resolve_kernel(LongBuffers lb, int nch, int keep,
                                                                       int* __restrict__ hist,
                                                                       int* __restrict__ cnt_out) {
  __shared__ LongShared sh;
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const LongRow lr = lb.row[row];
  const int c0 = lr.c0, above0 = lr.above0, nvis = lr.nvis;
  const uint32_t* cand = lb.cand + (size_t)row * nch * TC_CHUNK;
  // one round of loads: chunk t's candidate and above counts
  const int nc_t = t < nch ? min(max(lb.nc[(size_t)row * nch + t], 0), TC_CHUNK) : 0;
  const int na_t = t < nch ? lb.na[(size_t)row * nch + t] : 0;
  // leave the row's histogram zero for the next call (every chunk kernel has read it)
  int* hrow = hist + (size_t)row * HIST_REPLICAS * TK_HBINS;
  for (int i = t; i < HIST_REPLICAS * TK_HBINS; i += TL_THREADS) hrow[i] = 0;
  for (int i = t; i < 2048; i += TL_THREADS) sh.bins[i] = 0;
  if (t < 512) sh.bins2[t] = 0;
  if (t < TL_MAXCH) {
    sh.gt[t] = 0;
    sh.tie[t] = 0;
  }
  if (t == 0) {
    sh.sel[0] = -1;
    sh.sel2[0] = -1;
  }
  const bool resolve = c0 >= 0 && nvis > keep;  // block-uniform
  // the candidates' flat offsets, then the first TL_CAP candidates into LDS
  int n_all;
  const int coff_t = long_block_scan(nc_t, sh.wtot, &n_all) - nc_t;
  if (t < nch) sh.coff[t] = coff_t;
  __syncthreads();
  const int n_stage = resolve ? min(n_all, TL_CAP) : 0;
  for (int i = t; i < n_stage; i += TL_THREADS) {
    const int j = long_chunk_of(sh.coff, nch, i);
    sh.sk[i] = cand[(size_t)j * TC_CHUNK + (i - sh.coff[j])];
    sh.sj[i] = (uint16_t)j;
  }
  __syncthreads();
  // candidate i (flat order) and its chunk: staged, or read from the workspace past TL_CAP
  auto cand_at = [&](int i, int* j) __attribute__((always_inline)) {
    if (i < TL_CAP) {
      *j = sh.sj[i];
      return sh.sk[i];
    }
    *j = long_chunk_of(sh.coff, nch, i);
    return cand[(size_t)*j * TC_CHUNK + (i - sh.coff[*j])];
  };
  uint32_t T = 0u;
  int room = 0;
  if (resolve) {
    int need = keep - above0;
    int j;
    // pass A: bits 19 .. 9 of every candidate
    for (int i = t; i < n_all; i += TL_THREADS) atomicAdd(&sh.bins[(cand_at(i, &j) >> 9) & 2047u], 1);
    __syncthreads();
    int c1, above;
    long_find_bin(sh, sh.bins, sh.sel, 2048, need, &c1, &above);
    need -= above;
    const uint32_t pre = ((uint32_t)c0 << 11) | (uint32_t)c1;
    // pass B: bits 8 .. 0 of the candidates under the 23-bit prefix
    for (int i = t; i < n_all; i += TL_THREADS) {
      const uint32_t k = cand_at(i, &j);
      if ((k >> 9) == pre) atomicAdd(&sh.bins2[k & 511u], 1);
    }
    __syncthreads();
    int c2;
    long_find_bin(sh, sh.bins2, sh.sel2, 512, need, &c2, &above);
    T = (pre << 9) | (uint32_t)c2;
    room = max(need - above, 0);
    // per chunk: its candidates above T and equal to T
    for (int i = t; i < n_all; i += TL_THREADS) {
      const uint32_t k = cand_at(i, &j);
      if (k > T) atomicAdd(&sh.gt[j], 1);
      if (k == T) atomicAdd(&sh.tie[j], 1);
    }
  }
  __syncthreads();
  // chunk t (t < nch): the ties before it, its ties taken, its first output index
  const int tie_t = t < nch ? sh.tie[t] : 0;
  int tot;
  const int tie_before = long_block_scan(tie_t, sh.wtot, &tot) - tie_t;
  const int take_t = min(max(room - tie_before, 0), tie_t);
  const int sel_t = t < nch ? na_t + sh.gt[t] + take_t : 0;
  const int base_t = long_block_scan(sel_t, sh.wtot, &tot) - sel_t;
  if (t < nch) {
    lb.base[(size_t)row * nch + t] = base_t;
    lb.take[(size_t)row * nch + t] = take_t;
  }
  if (t == 0) {
    lb.row[row].T = T;
    cnt_out[row] = nvis < 0 ? 0 : (nvis < keep ? nvis : keep);
  }
}

template <bool VEC, bool ROWS>
__global__ __launch_bounds__(TC_THREADS) void topk_long_output_kernel(const float* __restrict__ scores, int stride,
                                                                      const int* __restrict__ len, int keep,
                                                                      int vis_only, LongBuffers lb, int nch,
                                                                      const int* __restrict__ cnt_in,
                                                                      int* __restrict__ idx_out, SlotOut so) {
  __shared__ ChunkShared sh;
  __shared__ int pg[WAVE];
  __shared__ int pg0s;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = level_len(len, row, 1, 1, stride);
  const int base = chunk * TC_CHUNK;
  const size_t ci = (size_t)row * nch + chunk;
  const uint32_t T = lb.row[row].T;
  const int out_base = lb.base[ci], room_here = lb.take[ci];
  const int pg_first = ROWS ? base / so.page_size : 0;
  int pgv = 0, pg0v = 0;
  if (ROWS) {
    pgv = so.table[(size_t)row * so.max_pages + min(pg_first + lane, so.max_pages - 1)];
    pg0v = so.table[(size_t)row * so.max_pages];
  }
  uint32_t key[2][4];
  load_chunk_keys<VEC>(scores + (size_t)row * stride, stride, L, base, vis_only, key);
  if (ROWS && wave == 0) {
    pg[lane] = safe_page(pgv, so.num_pages);
    if (lane == 0) pg0s = safe_page(pg0v, so.num_pages);
  }
  uint32_t mine[2], before[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t na = 0, nt = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      na += key[e][c] > T;
      nt += T != 0u && key[e][c] == T;
    }
    mine[e] = (na << 16) | nt;
  }
  chunk_prefix(mine, sh.blk, before);  // its barriers also order the page ids' LDS writes before their reads
  int* orow = idx_out + (size_t)row * keep;
  const int psh = ROWS ? page_shift_of(so.page_size) : 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    int a_before = (int)(before[e] >> 16), t_before = (int)(before[e] & 0xffffu);
    const int p0 = base + 4 * (TC_THREADS * e + t);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool a = key[e][c] > T;
      const bool ti = T != 0u && key[e][c] == T;
      const bool sel = a || (ti && t_before < room_here);
      const int o = out_base + a_before + (t_before < room_here ? t_before : room_here);
      if (sel && (unsigned)o < (unsigned)keep) {
        orow[o] = p0 + c;
        if (ROWS) {
          const int ps = so.page_size, p = p0 + c, pi = page_of(p, ps, psh);
          so.rows[(size_t)row * keep + o] = pg[min(pi - pg_first, WAVE - 1)] * ps + (p - pi * ps);
        }
      }
      a_before += a;
      t_before += ti;
    }
  }
  if (chunk == 0) {
    const int cnt_row = cnt_in[row];
    for (int i = cnt_row + t; i < keep; i += TC_THREADS) {
      orow[i] = 0;
      if (ROWS) so.rows[(size_t)row * keep + i] = pg0s * so.page_size;
    }
  }
}

// Sub-block maxima of each row: bm[row, j] = max of scores[row, j sub .. j sub + sub - 1] over positions < len.
__global__ void block_max_kernel(const float* __restrict__ scores, int stride, const int* __restrict__ len, int sub,
                                 int nb_stride, float* __restrict__ bm) {
  const int row = blockIdx.y;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= nb_stride) return;
  int L = stride;
  if (len) L = min(max(len[row], 0), stride);
  const float* s = scores + (size_t)row * stride;
  float m = NEG_INF;
  const int p0 = j * sub;
  for (int e = 0; e < sub; ++e) {
    const int p = p0 + e;
    if (p < L) m = fmaxf(m, s[p]);
  }
  bm[(size_t)row * nb_stride + j] = m;
}

// Candidate rows of the second level: the selected sub-blocks' scores in ascending sub-block order
// (NEG_INF past the count or past the row's length).
__global__ void gather_blocks_kernel(const float* __restrict__ scores, int stride, const int* __restrict__ len,
                                     int sub, const int* __restrict__ bidx, const int* __restrict__ bcnt, int keep,
                                     float* __restrict__ cand) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= keep * sub) return;
  int L = stride;
  if (len) L = min(max(len[row], 0), stride);
  const int k = i / sub, e = i - k * sub;
  float v = NEG_INF;
  if (k < bcnt[row]) {
    const int p = bidx[(size_t)row * keep + k] * sub + e;
    if (p < L) v = scores[(size_t)row * stride + p];
  }
  cand[(size_t)row * keep * sub + i] = v;
}

// The mask's background: NEG_INF, or with tail 0 for every token of a non-candidate score (score <= VISIBLE, the
// reference's `sel | ~vis`, trnrt/kernels/dsa_topk.py:89-93), kp tokens per score. all (keep >= P, dsa_topk.py:
// 103-105): 0 for every visible score too (every score when scores is null), and no scatter follows.
__global__ void topk_mask_fill_kernel(const float* __restrict__ scores, float* __restrict__ mask, int P, int kp,
                                      int tail, int all) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P * kp) return;
  const bool vis = scores == nullptr || scores[(size_t)row * P + i / kp] > VISIBLE;
  const bool taken = (all && vis) || (tail && !vis);
  mask[(size_t)row * P * kp + i] = taken ? 0.0f : NEG_INF;
}

// 0 for the kp tokens of every selected score.
__global__ void topk_mask_scatter_kernel(const int* __restrict__ idx, const int* __restrict__ cnt,
                                         float* __restrict__ mask, int keep, int P, int kp) {
  const int row = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < keep && k < cnt[row]) {
    const int p = idx[(size_t)row * keep + k];
    if ((unsigned)p < (unsigned)P)
      for (int t = 0; t < kp; ++t) mask[((size_t)row * P + p) * kp + t] = 0.0f;
  }
}

// gather_blocks_kernel with 16-byte loads and stores (sub a multiple of 4, rows 16-byte aligned): thread i moves
// scores 4 i .. 4 i + 3 of the candidate row.
__global__ void gather_blocks4_kernel(const float* __restrict__ scores, int stride, const int* __restrict__ len,
                                      int sub, const int* __restrict__ bidx, const int* __restrict__ bcnt, int keep,
                                      float* __restrict__ cand) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (4 * i >= keep * sub) return;
  int L = stride;
  if (len) L = min(max(len[row], 0), stride);
  const int k = (4 * i) / sub, e = 4 * i - k * sub;
  float4 v = make_float4(NEG_INF, NEG_INF, NEG_INF, NEG_INF);
  if (k < bcnt[row]) {
    const int p = bidx[(size_t)row * keep + k] * sub + e;
    if (p + 3 < L) {
      v = *reinterpret_cast<const float4*>(scores + (size_t)row * stride + p);
    } else {
      const float* sr = scores + (size_t)row * stride;
      v.x = p < L ? sr[p] : NEG_INF;
      v.y = p + 1 < L ? sr[p + 1] : NEG_INF;
      v.z = p + 2 < L ? sr[p + 2] : NEG_INF;
    }
  }
  reinterpret_cast<float4*>(cand + (size_t)row * keep * sub)[i] = v;
}

// Positions of a candidate row -> positions of the row it was gathered from (sub-blocks bidx of `sub` each).
__global__ void map_blocks_kernel(int* __restrict__ idx, const int* __restrict__ cnt, const int* __restrict__ bidx,
                                  int sub, int keep) {
  const int row = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < keep && k < cnt[row]) {
    const int p = idx[(size_t)row * keep + k];
    idx[(size_t)row * keep + k] = bidx[(size_t)row * keep + p / sub] * sub + p % sub;
  }
}

// The prefill selection's outputs in the reference's form (trnrt/kernels/dsa_long_select.py:494-528 `select`): the
// selected positions (through the selected sub-blocks bidx of `sub` each, when the rows were selected in two levels)
// as int64, 0 past the count; their scores, NEG_INF past the count; the count as int64. idx keeps the positions.
__global__ void select_out_kernel(int* __restrict__ idx, const int* __restrict__ cnt, const int* __restrict__ bidx,
                                  int sub, int keep, const float* __restrict__ scores, int stride,
                                  int64_t* __restrict__ pools, int64_t* __restrict__ cnt64, float* __restrict__ vals) {
  const int row = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= keep) return;
  const int c = cnt[row];
  const size_t o = (size_t)row * keep + k;
  int p = 0;
  float v = NEG_INF;
  if (k < c) {
    p = idx[o];
    if (bidx) p = bidx[(size_t)row * keep + p / sub] * sub + p % sub;
    p = min(max(p, 0), stride - 1);
    v = scores[(size_t)row * stride + p];
    idx[o] = p;
  }
  pools[o] = p;
  vals[o] = v;
  if (k == 0) cnt64[row] = c;
}

// One workgroup per row up to TOPK_FLAT_MAX scores; longer rows are selected in two levels, recursively.
constexpr int TOPK_FLAT_MAX = 4 * TR_MAXG * TR_THREADS;
constexpr int TOPK_LONG_KEEP_MAX = 8192;

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// The sub-block of the two-level selection of rows of n scores: a power of two near sqrt(n / keep), which balances
// the sub-block maxima (n / sub) against the candidates (keep sub).
static int topk_sub_block(long n, int keep) {
  int sub = 2;
  while ((long)sub * sub * 2 * keep <= n) sub *= 2;  // sub^2 keep <= n / 2 < (2 sub)^2 keep
  return sub;
}

// Recursion plan shared by the workspace size and the launch.
static bool topk_plan(long n, int keep) {
  if (n <= TOPK_FLAT_MAX) return true;
  if (keep > TOPK_LONG_KEEP_MAX) return false;
  const int sub = topk_sub_block(n, keep);
  const long nb = (n + sub - 1) / sub, nc = (long)keep * sub;
  // level 1 (the sub-block maxima) runs flat; level 2 (the candidates) may split again
  if (nb > TOPK_FLAT_MAX || nc >= n) return false;
  return topk_plan(nc, keep);
}

// Workspace of a selection: the first-level histograms [B, 4096] int (zero between calls), then the two-level
// buffers of rows longer than TOPK_FLAT_MAX (recursively).
static size_t topk_level_bytes(int B, long n, int keep) {
  if (n <= TOPK_FLAT_MAX) return 0;
  const int sub = topk_sub_block(n, keep);
  const long nb = (n + sub - 1) / sub, nc = (long)keep * sub;
  return up256((size_t)B * nb * 4) + up256((size_t)B * keep * 4) + up256((size_t)B * 4) + up256((size_t)B * nc * 4) +
         topk_level_bytes(B, nc, keep);
}

size_t topk_hist_bytes(int B) { return up256((size_t)B * HIST_REPLICAS * TK_HBINS * 4); }

// The region a workspace keeps at zero between calls: the barrier and status words (WS_SYNC_BYTES, the first bytes of
// every workspace: the status words excepted), then the histograms.
size_t topk_zero_bytes(int B) { return WS_SYNC_BYTES + topk_hist_bytes(B); }

static bool topk_long_ok(int B, long n);
static size_t topk_long_bytes(int B, long n);

size_t topk_workspace_bytes(int B, int max_len, int keep) {
  size_t rest = topk_level_bytes(B, max_len, keep);
  if (topk_long_ok(B, max_len)) {  // the long selection's buffers share the two-level selection's place
    const size_t l = topk_long_bytes(B, max_len);
    rest = l > rest ? l : rest;
  }
  return topk_zero_bytes(B) + up256((size_t)B * sizeof(RowMeta)) + up256((size_t)B * TC_MAXCH * TC_CHUNK * 4) + rest;
}

bool topk_supported(int max_len, int keep, int vis_only) {
  if (keep < 1) return false;
  if (max_len <= TOPK_FLAT_MAX) return true;
  return vis_only && topk_plan(max_len, keep);
}

// The flat selection's buffers inside the top-k workspace: past the barrier and status words, the first-level
// histograms [B, 4096] (zero between calls), then the per-row meta and the candidate lists of the chunked kernels.
struct TopkBuffers {
  int* hist;
  RowMeta* meta;
  uint32_t* ckey;
};

// The prefill selection's outputs (select_out_kernel).
struct SelectOut {
  int64_t* pools;
  int64_t* cnt;
  float* vals;
};

template <int G, bool VEC>
static hipError_t launch_topk_row(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                  int keep, int vis_only, int* hist, bool hist_ready, int* idx, int* cnt,
                                  const SlotOut& so, int B, hipStream_t s) {
  const dim3 grid(B), block(TR_THREADS);
  if (so.rows)
    return hist_ready ? launch("topk_row_kernel", topk_row_kernel<G, true, VEC, true>, grid, block, s, scores, stride,
                               len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, IndOut{})
                      : launch("topk_row_kernel", topk_row_kernel<G, false, VEC, true>, grid, block, s, scores,
                               stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, IndOut{});
  return hist_ready ? launch("topk_row_kernel", topk_row_kernel<G, true, VEC, false>, grid, block, s, scores, stride,
                             len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, IndOut{})
                    : launch("topk_row_kernel", topk_row_kernel<G, false, VEC, false>, grid, block, s, scores, stride,
                             len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, IndOut{});
}

// Many rows (a prefill chunk's queries, the two-level selection's levels): one workgroup per row holds the whole row
// (up to 8 float4 groups per thread, 32,768 scores) and selects it in one kernel, reading it once; the chunked form
// spreads few long rows over many CUs instead.
constexpr int TOPK_MANY_ROWS = 512;

template <int G, bool VEC>
static hipError_t launch_topk_row_plain(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                        int keep, int vis_only, int* hist, int* idx, int* cnt, const SlotOut& so,
                                        int B, hipStream_t s, const IndOut* out64) {
  if (out64)  // the reference's outputs written directly (IndOut's pools, cnt, vals)
    return launch("topk_row_kernel", topk_row_kernel<G, false, VEC, false, false, true>, dim3(B), dim3(TR_THREADS), s,
                  scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, *out64);
  return launch("topk_row_kernel", topk_row_kernel<G, false, VEC, false>, dim3(B), dim3(TR_THREADS), s, scores,
                stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so, IndOut{});
}

template <bool VEC>
static hipError_t launch_topk_many_rows(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                        int max_len, int keep, int vis_only, int* hist, int* idx, int* cnt,
                                        const SlotOut& so, int B, hipStream_t s, const IndOut* out64 = nullptr) {
  switch ((max_len + 4 * TR_THREADS - 1) / (4 * TR_THREADS)) {
    case 1:
      return launch_topk_row_plain<1, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
    case 2:
      return launch_topk_row_plain<2, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
    case 3:
      return launch_topk_row_plain<3, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
    case 4:
      return launch_topk_row_plain<4, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
    case 5:
    case 6:
      return launch_topk_row_plain<6, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
    default:
      return launch_topk_row_plain<8, VEC>(scores, stride, len, len_div, len_mul, keep, vis_only, hist, idx, cnt, so,
                                           B, s, out64);
  }
}

template <int G>
static hipError_t launch_topk_ind_g(int nc, int keep, int vis_only, const IndOut& io, int B, hipStream_t s) {
  const SlotOut none = {nullptr, 0, 0, 0, nullptr};
  return launch("topk_row_kernel", topk_row_kernel<G, false, true, false, true>, dim3(B), dim3(TR_THREADS), s,
                nullptr, nc, nullptr, 1, 1, keep, vis_only, nullptr, nullptr, nullptr, none, io);
}

// The IND second level over nc <= TOPK_FLAT_MAX candidates per row.
static hipError_t launch_topk_ind(int nc, int keep, int vis_only, const IndOut& io, int B, hipStream_t s) {
  switch ((nc + 4 * TR_THREADS - 1) / (4 * TR_THREADS)) {
    case 1:
      return launch_topk_ind_g<1>(nc, keep, vis_only, io, B, s);
    case 2:
      return launch_topk_ind_g<2>(nc, keep, vis_only, io, B, s);
    case 3:
    case 4:
      return launch_topk_ind_g<4>(nc, keep, vis_only, io, B, s);
    default:
      return launch_topk_ind_g<8>(nc, keep, vis_only, io, B, s);
  }
}

template <bool VEC>
static hipError_t launch_topk_chunked(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                      int nch, int keep, int vis_only, int* idx, int* cnt, const TopkBuffers& tb,
                                      bool hist_ready, const SlotOut& so, int B, hipStream_t s) {
  hipError_t e;
  if (!hist_ready) {
    e = launch("topk_hist_kernel", topk_hist_kernel, dim3(nch, B), dim3(TKH_THREADS), s, scores, stride, len, len_div,
               len_mul, vis_only, tb.hist);
    if (e != hipSuccess) return e;
  }
  e = launch("topk_chunk_kernel", topk_chunk_kernel<VEC>, dim3(nch, B), dim3(TC_THREADS), s, scores, stride, len,
             len_div, len_mul, keep, vis_only, tb.hist, tb.meta, tb.ckey);
  if (e != hipSuccess) return e;
  if (so.rows)
    return launch("topk_output_kernel", topk_output_kernel<VEC, true>, dim3(nch, B), dim3(TC_THREADS), s, scores,
                  stride, len, len_div, len_mul, keep, vis_only, nch, tb.hist, tb.meta, tb.ckey, idx, cnt, so);
  return launch("topk_output_kernel", topk_output_kernel<VEC, false>, dim3(nch, B), dim3(TC_THREADS), s, scores,
                stride, len, len_div, len_mul, keep, vis_only, nch, tb.hist, tb.meta, tb.ckey, idx, cnt, so);
}

// The flat selection of rows of at most max_len <= TOPK_FLAT_MAX scores: one workgroup per row up to 4096 scores,
// the chunked kernels above that.
static hipError_t launch_topk_level(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                    int max_len, int keep, int vis_only, int* idx, int* cnt, const TopkBuffers& tb,
                                    bool hist_ready, const SlotOut& so, int B, hipStream_t s) {
  const bool vec = (stride & 3) == 0 && stride >= 4;
  if (max_len <= 4 * TR_THREADS)
    return vec ? launch_topk_row<1, true>(scores, stride, len, len_div, len_mul, keep, vis_only, tb.hist, hist_ready,
                                          idx, cnt, so, B, s)
               : launch_topk_row<1, false>(scores, stride, len, len_div, len_mul, keep, vis_only, tb.hist, hist_ready,
                                           idx, cnt, so, B, s);
  if (max_len > TC_MAXCH * TC_CHUNK) return hipErrorInvalidValue;
  // the first-level histogram ready (the fused indexer's) and rows of at most 8192 scores: one workgroup per row,
  // one kernel (measured at 8 rows: 7.3 us against 4.6 + 5.8 us for the chunked pair at 8192 scores, but 20.1 us
  // against 4.3 + 7.4 us at 32768, where one CU per row is the bound)
  if (hist_ready && max_len <= 8 * TR_THREADS &&
      (!so.rows || (max_len + so.page_size - 1) / so.page_size <= TR_THREADS))
    return vec ? launch_topk_row<2, true>(scores, stride, len, len_div, len_mul, keep, vis_only, tb.hist, true, idx,
                                          cnt, so, B, s)
               : launch_topk_row<2, false>(scores, stride, len, len_div, len_mul, keep, vis_only, tb.hist, true, idx,
                                           cnt, so, B, s);
  if (B >= TOPK_MANY_ROWS && !hist_ready && !so.rows)
    return vec ? launch_topk_many_rows<true>(scores, stride, len, len_div, len_mul, max_len, keep, vis_only, tb.hist,
                                             idx, cnt, so, B, s)
               : launch_topk_many_rows<false>(scores, stride, len, len_div, len_mul, max_len, keep, vis_only, tb.hist,
                                              idx, cnt, so, B, s);
  const int nch = (max_len + TC_CHUNK - 1) / TC_CHUNK;
  return vec ? launch_topk_chunked<true>(scores, stride, len, len_div, len_mul, nch, keep, vis_only, idx, cnt, tb,
                                         hist_ready, so, B, s)
             : launch_topk_chunked<false>(scores, stride, len, len_div, len_mul, nch, keep, vis_only, idx, cnt, tb,
                                          hist_ready, so, B, s);
}

static size_t topk_long_bytes(int B, long n) {
  const size_t nch = (size_t)((n + TC_CHUNK - 1) / TC_CHUNK);
  return up256((size_t)B * sizeof(LongRow)) + 4 * up256((size_t)B * nch * 4) + up256((size_t)B * nch * TC_CHUNK * 4);
}

static LongBuffers topk_long_buffers(char* p, int B, int nch) {
  LongBuffers lb;
  lb.row = reinterpret_cast<LongRow*>(p);
  p += up256((size_t)B * sizeof(LongRow));
  int** arrs[4] = {&lb.na, &lb.nc, &lb.base, &lb.take};
  for (int** a : arrs) {
    *a = reinterpret_cast<int*>(p);
    p += up256((size_t)B * nch * 4);
  }
  lb.cand = reinterpret_cast<uint32_t*>(p);
  return lb;
}

// Whether the long selection takes rows of up to n scores in a batch of B rows (few rows: many rows take the
// one-workgroup-per-row kernels).
static bool topk_long_ok(int B, long n) {
  return n > TOPK_FLAT_MAX && B < TOPK_MANY_ROWS && (n + TC_CHUNK - 1) / TC_CHUNK <= TL_MAXCH;
}

template <bool VEC>
static hipError_t launch_topk_long_v(const float* scores, int stride, const int* len, long n, int keep, int vis_only,
                                     int* hist, bool hist_ready, char* p, int* idx, int* cnt, const SlotOut& so,
                                     int B, hipStream_t s) {
  const int nch = (int)((n + TC_CHUNK - 1) / TC_CHUNK);
  const LongBuffers lb = topk_long_buffers(p, B, nch);
  hipError_t e;
  if (!hist_ready) {
    e = launch("topk_hist_kernel", topk_hist_kernel, dim3(nch, B), dim3(TKH_THREADS), s, scores, stride, len, 1, 1,
               vis_only, hist);
    if (e != hipSuccess) return e;
  }
  e = launch("topk_long_chunk_kernel", topk_long_chunk_kernel<VEC>, dim3(nch, B), dim3(TC_THREADS), s, scores, stride,
             len, keep, vis_only, hist, lb, nch);
  if (e != hipSuccess) return e;
  e = launch("topk_long_resolve_kernel", topk_long_resolve_kernel, dim3(B), dim3(TL_THREADS), s, lb, nch, keep, hist,
             cnt);
  if (e != hipSuccess) return e;
  if (so.rows)
    return launch("topk_long_output_kernel", topk_long_output_kernel<VEC, true>, dim3(nch, B), dim3(TC_THREADS), s,
                  scores, stride, len, keep, vis_only, lb, nch, cnt, idx, so);
  return launch("topk_long_output_kernel", topk_long_output_kernel<VEC, false>, dim3(nch, B), dim3(TC_THREADS), s,
                scores, stride, len, keep, vis_only, lb, nch, cnt, idx, so);
}

// Selection over rows of `stride` scores whose lengths are len[row] (len_div / len_mul as in level_len), n an upper
// bound of the lengths.
static hipError_t topk_rows(const float* scores, int stride, const int* len, int len_div, int len_mul, long n,
                            int keep, int vis_only, int* idx, int* cnt, const TopkBuffers& tb, bool hist_ready,
                            char* ws, int B, hipStream_t s, bool bm_ready = false, const SelectOut* out = nullptr) {
  const SlotOut none = {nullptr, 0, 0, 0, nullptr};
  if (n <= TOPK_FLAT_MAX) {
    if (out && B >= TOPK_MANY_ROWS && !hist_ready && n > 4 * TR_THREADS) {
      // many rows: the one-workgroup-per-row kernel writes the reference's outputs itself
      const IndOut io = {nullptr, 0, nullptr, nullptr, nullptr, 0, out->pools, out->cnt, out->vals};
      return (stride & 3) == 0 ? launch_topk_many_rows<true>(scores, stride, len, len_div, len_mul, (int)n, keep,
                                                             vis_only, tb.hist, idx, cnt, none, B, s, &io)
                               : launch_topk_many_rows<false>(scores, stride, len, len_div, len_mul, (int)n, keep,
                                                              vis_only, tb.hist, idx, cnt, none, B, s, &io);
    }
    hipError_t e = launch_topk_level(scores, stride, len, len_div, len_mul, (int)n, keep, vis_only, idx, cnt, tb,
                                     hist_ready, none, B, s);
    if (e != hipSuccess || !out) return e;
    return launch("select_out_kernel", select_out_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt,
                  nullptr, 1, keep, scores, stride, out->pools, out->cnt, out->vals);
  }
  if (len_div != 1 || len_mul != 1) return hipErrorInvalidValue;  // only flat rows are split
  const int sub = topk_sub_block(n, keep);
  const int nb = (int)((n + sub - 1) / sub), nc = keep * sub;
  float* bm = reinterpret_cast<float*>(ws);
  ws += up256((size_t)B * nb * 4);
  int* bidx = reinterpret_cast<int*>(ws);
  ws += up256((size_t)B * keep * 4);
  int* bcnt = reinterpret_cast<int*>(ws);
  ws += up256((size_t)B * 4);
  float* cand = reinterpret_cast<float*>(ws);
  ws += up256((size_t)B * nc * 4);
  hipError_t e = hipSuccess;
  if (!bm_ready) {  // else the indexer wrote the maxima there (topk_bm_buffer)
    e = launch("block_max_kernel", block_max_kernel, dim3((nb + 255) / 256, B), dim3(256), s, scores, stride, len, sub,
               nb, bm);
    if (e != hipSuccess) return e;
  }
  // level 1: the top-keep sub-blocks (ceil(len / sub) maxima per row)
  if (nb > TOPK_FLAT_MAX) return hipErrorInvalidValue;  // excluded by topk_plan
  e = launch_topk_level(bm, nb, len, sub, 1, nb, keep, vis_only, bidx, bcnt, tb, false, none, B, s);
  if (e != hipSuccess) return e;
  // many rows with their outputs in the reference's form: the second level reads the selected sub-blocks in place
  // and writes those outputs (no candidate rows, no separate mapping)
  if (out && B >= TOPK_MANY_ROWS && nc <= TOPK_FLAT_MAX && (sub & 3) == 0 && (stride & 3) == 0 && len) {
    const IndOut io = {scores, stride, len, bidx, bcnt, sub, out->pools, out->cnt, out->vals};
    return launch_topk_ind(nc, keep, vis_only, io, B, s);
  }
  if ((sub & 3) == 0 && (stride & 3) == 0)
    e = launch("gather_blocks_kernel", gather_blocks4_kernel, dim3((nc / 4 + 255) / 256, B), dim3(256), s, scores,
               stride, len, sub, bidx, bcnt, keep, cand);
  else
    e = launch("gather_blocks_kernel", gather_blocks_kernel, dim3((nc + 255) / 256, B), dim3(256), s, scores, stride,
               len, sub, bidx, bcnt, keep, cand);
  if (e != hipSuccess) return e;
  // level 2: the top-keep of the selected sub-blocks' scores in position order (NEG_INF past their count)
  e = topk_rows(cand, nc, nullptr, 1, 1, nc, keep, vis_only, idx, cnt, tb, false, ws, B, s);
  if (e != hipSuccess) return e;
  if (out)
    return launch("select_out_kernel", select_out_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, bidx,
                  sub, keep, scores, stride, out->pools, out->cnt, out->vals);
  return launch("map_blocks_kernel", map_blocks_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, bidx,
                sub, keep);
}

// ws: topk_workspace_bytes(B, max_len, keep) bytes whose histogram region is zero; hist_ready: the histogram of the
// rows is already accumulated there (by the indexer), so the first level does not build it. rows_out (flat rows
// only, else null): also the cache slot of each selected position through the page table. bm_ready (rows longer than
// TOPK_FLAT_MAX): the first level's sub-block maxima are already in topk_bm_buffer(ws, B) (the indexer wrote them).
hipError_t launch_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                       int max_len, int keep, int vis_only, bool hist_ready, const int* table, int max_pages,
                       int page_size, int num_pages, int* rows_out, hipStream_t s, bool bm_ready) {
  char* p = static_cast<char*>(ws);
  const bool long_rows = topk_long_ok(B, max_len);
  if ((hist_ready || rows_out) && max_len > TOPK_FLAT_MAX && !long_rows) return hipErrorInvalidValue;
  if (rows_out && (!table || page_size < 32 || max_pages < 1 || num_pages < 1)) return hipErrorInvalidValue;
  TopkBuffers tb;
  tb.hist = ws_hist(p);
  p += topk_zero_bytes(B);
  tb.meta = reinterpret_cast<RowMeta*>(p);
  p += up256((size_t)B * sizeof(RowMeta));
  tb.ckey = reinterpret_cast<uint32_t*>(p);
  p += up256((size_t)B * TC_MAXCH * TC_CHUNK * 4);
  if (long_rows && !bm_ready) {
    const SlotOut so = {table, max_pages, page_size, num_pages, rows_out};
    return (stride & 3) == 0 ? launch_topk_long_v<true>(scores, stride, len, max_len, keep, vis_only, tb.hist,
                                                        hist_ready, p, idx, cnt, so, B, s)
                             : launch_topk_long_v<false>(scores, stride, len, max_len, keep, vis_only, tb.hist,
                                                         hist_ready, p, idx, cnt, so, B, s);
  }
  if (rows_out) {
    const SlotOut so = {table, max_pages, page_size, num_pages, rows_out};
    return launch_topk_level(scores, stride, len, 1, 1, max_len, keep, vis_only, idx, cnt, tb, hist_ready, so, B, s);
  }
  return topk_rows(scores, stride, len, 1, 1, max_len, keep, vis_only, idx, cnt, tb, hist_ready, p, B, s,
                   bm_ready && max_len > TOPK_FLAT_MAX);
}

// Whether a batch of B rows of up to n scores takes the long selection (then the first-level histogram can come from
// the indexer, and the slot output is available).
bool topk_long_rows(int B, long n) { return topk_long_ok(B, n); }

// The sub-block size of the first level of rows of n scores (a power of two), or 0 when they are selected flat.
int topk_two_level_sub(long n, int keep) { return n <= TOPK_FLAT_MAX ? 0 : topk_sub_block(n, keep); }

// Where the first level's sub-block maxima [B, ceil(n / sub)] live in a top-k workspace: written there by a producer
// (the prefill indexer), they let launch_prefill_topk skip block_max_kernel.
float* topk_bm_buffer(void* ws, int B) {
  return reinterpret_cast<float*>(static_cast<char*>(ws) + topk_zero_bytes(B) + up256((size_t)B * sizeof(RowMeta)) +
                                  up256((size_t)B * TC_MAXCH * TC_CHUNK * 4));
}

// The prefill chunk's selection of rows of n <= stride scores (lengths len): the exact top-keep of each row, written
// as the reference's (pools int64, cnt int64, vals) through idx / cnt (int32 [B, keep], [B]); bm_ready: the first
// level's sub-block maxima are already in topk_bm_buffer(ws).
hipError_t launch_prefill_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                               int n, int keep, bool bm_ready, int64_t* pools, int64_t* cnt64, float* vals,
                               hipStream_t s) {
  char* p = static_cast<char*>(ws);
  TopkBuffers tb;
  tb.hist = ws_hist(p);
  p += topk_zero_bytes(B);
  tb.meta = reinterpret_cast<RowMeta*>(p);
  p += up256((size_t)B * sizeof(RowMeta));
  tb.ckey = reinterpret_cast<uint32_t*>(p);
  p += up256((size_t)B * TC_MAXCH * TC_CHUNK * 4);
  const SelectOut out = {pools, cnt64, vals};
  return topk_rows(scores, stride, len, 1, 1, n, keep, 1, idx, cnt, tb, false, p, B, s, bm_ready, &out);
}

// The prefill selection of one tile of rows through the one-workgroup-per-row kernels only (whatever the tile's row
// count), so that it needs none of the chunked kernels' buffers (histograms, row meta, candidate keys). The plan of
// rows of at most n scores in rows of `stride`: 0 flat (n <= TOPK_FLAT_MAX: one kernel writing the reference's
// outputs); sub in {4, 8, 16} two levels, the first over the sub-block maxima [rows, ceil(n / sub)] that the indexer
// wrote, the second reading the selected sub-blocks' scores in place (IND); -1 neither (launch_prefill_topk's generic
// form over a workspace of topk_workspace_bytes).
int prefill_tile_plan(long n, int stride, int keep) {
  if (n <= TOPK_FLAT_MAX) return 0;
  if (keep > TOPK_LONG_KEEP_MAX) return -1;
  const int sub = topk_sub_block(n, keep);
  const long nb = (n + sub - 1) / sub, nc = (long)keep * sub;
  if (sub < 4 || sub > 16 || (stride & 3) || nb > TOPK_FLAT_MAX || nc > TOPK_FLAT_MAX || nc >= n) return -1;
  return sub;
}

// One tile (T rows) of a plan >= 0 selection: scores [T, stride] with lengths len[T]; plan > 0: bm [T, nb] the
// sub-block maxima (row stride nb = ceil(n / sub)), bidx [T, keep] and bcnt [T] the first level's output. Writes
// pools / cnt64 / vals [T, ...] as launch_prefill_topk does.
hipError_t launch_prefill_tile_topk(const float* scores, int stride, const int* len, long n, int keep,
                                    const float* bm, int* bidx, int* bcnt, int64_t* pools, int64_t* cnt64,
                                    float* vals, int T, hipStream_t s) {
  const SlotOut none = {nullptr, 0, 0, 0, nullptr};
  const int plan = prefill_tile_plan(n, stride, keep);
  if (plan < 0) return hipErrorInvalidValue;
  if (plan == 0) {
    const IndOut io = {nullptr, 0, nullptr, nullptr, nullptr, 0, pools, cnt64, vals};
    return (stride & 3) == 0 ? launch_topk_many_rows<true>(scores, stride, len, 1, 1, (int)n, keep, 1, nullptr,
                                                           nullptr, nullptr, none, T, s, &io)
                             : launch_topk_many_rows<false>(scores, stride, len, 1, 1, (int)n, keep, 1, nullptr,
                                                            nullptr, nullptr, none, T, s, &io);
  }
  const int sub = plan, nb = (int)((n + sub - 1) / sub), nc = keep * sub;
  // level 1: the top-keep sub-blocks of each row (ceil(len / sub) maxima)
  hipError_t e = (nb & 3) == 0 ? launch_topk_many_rows<true>(bm, nb, len, sub, 1, nb, keep, 1, nullptr, bidx, bcnt,
                                                             none, T, s)
                               : launch_topk_many_rows<false>(bm, nb, len, sub, 1, nb, keep, 1, nullptr, bidx, bcnt,
                                                              none, T, s);
  if (e != hipSuccess) return e;
  const IndOut io = {scores, stride, len, bidx, bcnt, sub, pools, cnt64, vals};
  return launch_topk_ind(nc, keep, 1, io, T, s);
}

// Zero-fills a workspace (a kernel, not a memset, so that callers may capture it in a graph).
__global__ void fill_zero_kernel(uint4* __restrict__ p, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
  const size_t n16 = bytes / 16;
  if (n16) {
    const int grid = (int)((n16 + 255) / 256 < 4096 ? (n16 + 255) / 256 : 4096);
    launch("fill_zero_kernel", fill_zero_kernel, dim3(grid), dim3(256), s, static_cast<uint4*>(p), n16);
  }
  return hipGetLastError();
}

hipError_t launch_topk_mask(const int* idx, const int* cnt, const float* scores, float* mask, int B, int keep, int P,
                            int kp, int tail, hipStream_t s) {
  const int all = idx == nullptr;
  hipError_t e = launch("topk_mask_fill_kernel", topk_mask_fill_kernel, dim3((P * kp + 255) / 256, B), dim3(256), s,
                        scores, mask, P, kp, tail, all);
  if (e != hipSuccess || all) return e;
  return launch("topk_mask_scatter_kernel", topk_mask_scatter_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx,
                cnt, mask, keep, P, kp);
}

}  // namespace dsa
