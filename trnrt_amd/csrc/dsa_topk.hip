// Exact per-row top-k for gfx950 (the selection rule of trnrt/models/dsa_select.py:10-38 and
// trnrt/kernels/dsa_topk.py:10-40, output form of trnrt/models/dsa_long.py:94-112 `_ascending`):
// per row, the `keep` largest selectable scores; every selected score >= every unselected one; among the scores
// equal to the keep-th largest, the lowest positions; only scores > VISIBLE are selectable (vis_only); a row with
// fewer selectable scores than keep selects all of them. Output: the positions in ascending order plus the count.
//
// One workgroup of 1024 threads owns a row of up to 1024 E scores, E consecutive positions per thread, held in
// registers as order-preserving integer keys (dsa_common.h order_key), so every comparison is exact (the reference's
// radix search over the threshold's bit pattern, dsa_topk.py:19-26, is exact for the same reason).
//
// The threshold search narrows a key interval [lo, hi] that contains the keep-th largest key, with `need` = its rank
// from the top inside the interval, by histograms in LDS:
//   - first pass: 2048 bins linear in VALUE over [min, max] of the row (a monotone binning, so each bin is a key
//     interval; it spreads the bell-shaped indexer scores over many bins, where the leading key bits would put most
//     of them into a few);
//   - then passes over the low bits of (key - lo), 11 bits at a time, until lo == hi = the threshold T.
// A pass counts only the keys inside the current interval, so the later passes touch a few keys.
// Selection: key > T, plus the first `room` = keep - #(key > T) keys equal to T by position (a block-wide prefix
// count over the tied keys in position order), written in position order by a block-wide prefix count.
//
// Longer rows go through the reference's two-level exact selection (trnrt/models/dsa_long.py:26-42, 114-132):
// sub-block maxima, the top-keep sub-blocks, and the top-keep of their elements in position order.
#include "dsa_common.h"

namespace dsa {

constexpr int TK_THREADS = 1024;
constexpr int TK_WAVES = TK_THREADS / WAVE;
constexpr int TK_BINS = 2048;   // bins of a refinement pass (11 key bits)
constexpr int TK_BITS = 11;
constexpr int TK_HSHIFT = 20;   // first level: the top 12 bits of the order key
constexpr int TK_HBINS = 4096;
constexpr int TKH_THREADS = 256;  // histogram kernel: 8 scores per thread, 2048 per workgroup
constexpr int TKH_CHUNK = TKH_THREADS * 8;

struct TopkShared {
  int hist[TK_BINS];
  uint32_t scan_tot[TK_WAVES];
  int sel_bin;
  int sel_above;
};

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

__device__ __forceinline__ uint32_t select_key(float v, int vis_only) {
  return (!vis_only || v > VISIBLE) ? order_key(v) : 0u;
}

// Block-wide exclusive prefix sum (thread order) of a uint32 per thread; returns it and the total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, TopkShared& sh, uint32_t* total) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  const uint32_t inc = (uint32_t)wave_incl_scan((int)v);
  if (lane == WAVE - 1) sh.scan_tot[wave] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) {
    const uint32_t x = sh.scan_tot[i];
    before += i < wave ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Exclusive suffix sum (reverse thread order): the sum of v over the threads above this one, and the total.
__device__ __forceinline__ int block_excl_suffix(int v, TopkShared& sh, int* total) {
  const int rt = TK_THREADS - 1 - (int)threadIdx.x;  // reversed id: its wave is 15 - wave, its lane 63 - lane
  const int wave = rt / WAVE, lane = rt & (WAVE - 1);
  int inc = v;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int x = __shfl_down(inc, o, WAVE);  // the thread o above has reversed lane - o
    if (lane >= o) inc += x;
  }
  if (lane == WAVE - 1) sh.scan_tot[wave] = (uint32_t)inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) {
    const int x = (int)sh.scan_tot[i];
    before += i < wave ? x : 0;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

__device__ __forceinline__ int bit_length(uint32_t x) { return x ? 32 - __clz(x) : 0; }

// First level of a selection: the histogram of the top 12 bits of the selectable keys of each row, accumulated into
// hist[row, 4096] (zero before; the select kernel zeroes it again after reading). 2048 scores per workgroup.
__global__ __launch_bounds__(TKH_THREADS) void topk_hist_kernel(const float* __restrict__ scores, int stride,
                                                                const int* __restrict__ len, int len_div,
                                                                int len_mul, int vis_only, int* __restrict__ hist) {
  __shared__ int h[TK_HBINS];
  const int row = blockIdx.y;
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = blockIdx.x * TKH_CHUNK;
  if (base >= L) return;
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
  int* hrow = hist + (size_t)row * TK_HBINS;
  for (int i = threadIdx.x; i < TK_HBINS; i += TKH_THREADS) {
    const int c = h[i];
    if (c) atomicAdd(&hrow[i], c);
  }
}

__device__ __forceinline__ uint64_t lanes_below() {
  const int lane = threadIdx.x & (WAVE - 1);
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// The flat selection of rows of up to TS_MAXCH x 2048 scores, spread over workgroups of 2048 scores (chunks), in two
// kernels with no waiting between workgroups:
//   topk_chunk_kernel:  from the row's first-level histogram the threshold's 12-bit bin c0 (every chunk computes it);
//                       per chunk the count of keys in bins above c0 and the keys of bin c0 (the candidates, a few
//                       hundred per row for indexer scores), written in position order (so list order ranks ties);
//   topk_output_kernel: every chunk loads the row's candidates (thread t the t-th of each chunk), two histogram
//                       passes over their low key bits give the exact threshold T and the number of keys equal to T
//                       to take (lowest positions first), the chunk's output base follows from the per-chunk counts,
//                       and the chunk writes its selected positions in order.
// Thread t holds the float4 groups e = 0, 1 at chunk positions 4 (256 e + t) .. + 3 (coalesced loads), so group e
// of wave w is the contiguous block of 256 positions 1024 e + 256 w .. of the chunk.
constexpr int TS_THREADS = 256;
constexpr int TS_WAVES = TS_THREADS / WAVE;
constexpr int TS_G = 2;
constexpr int TS_CHUNK = TS_THREADS * 4 * TS_G;  // 2048
constexpr int TS_MAXCH = 16;                     // rows up to 32768 scores

struct RowMeta {
  int c0;      // the threshold's 12-bit bin (-1: every selectable key is selected)
  int above0;  // selectable keys in bins above c0
  int nvis;    // selectable keys of the row
  int pad;
  int n_a[TS_MAXCH];  // per chunk: keys in bins above c0
  int n_c[TS_MAXCH];  // per chunk: keys in bin c0
};

__device__ __forceinline__ void load_chunk_keys(const float* srow, int L, int base, bool vec, int vis_only,
                                                uint32_t (&key)[TS_G][4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    const int p = base + 4 * (TS_THREADS * e + t);
    if (vec && p + 4 <= L) {
      const float4 v = *reinterpret_cast<const float4*>(srow + p);
      key[e][0] = select_key(v.x, vis_only);
      key[e][1] = select_key(v.y, vis_only);
      key[e][2] = select_key(v.z, vis_only);
      key[e][3] = select_key(v.w, vis_only);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) key[e][c] = (p + c < L) ? select_key(srow[p + c], vis_only) : 0u;
    }
  }
}

// Exclusive prefix over the (e, wave) blocks of per-block counts (packed hi / lo 16 bits), in position order.
__device__ __forceinline__ void block_bases(uint32_t (&cnt)[TS_G], uint32_t* blk, uint32_t (&base)[TS_G]) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  if (lane == 0)
#pragma unroll
    for (int e = 0; e < TS_G; ++e) blk[e * TS_WAVES + wave] = cnt[e];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    uint32_t acc = 0;
    const int me = e * TS_WAVES + wave;
#pragma unroll
    for (int i = 0; i < TS_G * TS_WAVES; ++i) acc += i < me ? blk[i] : 0u;
    base[e] = acc;
  }
  __syncthreads();
}

struct ChunkShared {
  int bins[TS_THREADS];  // per thread: its 16 bins' sum, for the suffix scan
  uint32_t blk[TS_G * TS_WAVES];
  int c0, above0;
};

__global__ __launch_bounds__(TS_THREADS) void topk_chunk_kernel(const float* __restrict__ scores, int stride,
                                                                const int* __restrict__ len, int len_div,
                                                                int len_mul, int keep, int vis_only,
                                                                const int* __restrict__ hist,
                                                                RowMeta* __restrict__ meta,
                                                                uint32_t* __restrict__ ckey) {
  __shared__ ChunkShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, lane = t & (WAVE - 1);
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = chunk * TS_CHUNK;
  const int* hrow = hist + (size_t)row * TK_HBINS;
  int4 hv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) hv[i] = *reinterpret_cast<const int4*>(hrow + 16 * t + 4 * i);
  uint32_t key[TS_G][4];
  load_chunk_keys(scores + (size_t)row * stride, L, base, (stride & 3) == 0, vis_only, key);

  // suffix sums of the 16-bin groups (thread t: bins 16 t .. 16 t + 15), every thread its own exclusive suffix
  int hb[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[4 * i] = hv[i].x;
    hb[4 * i + 1] = hv[i].y;
    hb[4 * i + 2] = hv[i].z;
    hb[4 * i + 3] = hv[i].w;
  }
  int mine = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) mine += hb[i];
  if (t == 0) {
    sh.c0 = -1;
    sh.above0 = 0;
  }
  int inc = mine;  // suffix inside the wave: lanes >= this one
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int x = __shfl_down(inc, o, WAVE);
    if (lane + o < WAVE) inc += x;
  }
  if (lane == 0) sh.bins[t / WAVE] = inc;  // the wave's total
  __syncthreads();
  int suf = inc - mine, nvis = 0;
#pragma unroll
  for (int i = 0; i < TS_WAVES; ++i) {
    const int x = sh.bins[i];
    suf += i > t / WAVE ? x : 0;
    nvis += x;
  }
  if (nvis > keep && suf < keep && suf + mine >= keep) {
#pragma unroll
    for (int i = 15; i >= 0; --i) {
      if (suf < keep && suf + hb[i] >= keep) {
        sh.c0 = 16 * t + i;
        sh.above0 = suf;
      }
      suf += hb[i];
    }
  }
  __syncthreads();
  const int c0 = sh.c0;  // -1: at most keep selectable keys, every one is selected
  if (chunk == 0 && t == 0) {
    meta[row].c0 = c0;
    meta[row].above0 = sh.above0;
    meta[row].nvis = nvis;
  }
  // classification: above c0, or in c0 (a candidate); the candidates in position order
  const uint64_t below = lanes_below();
  uint64_t cm[TS_G][4];
  uint32_t cnt[TS_G], na = 0;
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    cnt[e] = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = key[e][c];
      const int bin = (int)(k >> TK_HSHIFT);
      na += __popcll(__ballot(k != 0 && bin > c0));
      cm[e][c] = __ballot(k != 0 && bin == c0);
      cnt[e] += __popcll(cm[e][c]);
    }
  }
  uint32_t bb[TS_G];
  block_bases(cnt, sh.blk, bb);
  uint32_t* krow = ckey + ((size_t)row * TS_MAXCH + chunk) * TS_CHUNK;
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    int o = (int)bb[e];
#pragma unroll
    for (int c = 0; c < 4; ++c) o += __popcll(cm[e][c] & below);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((cm[e][c] >> lane) & 1ull) krow[o++] = key[e][c];
    }
  }
  // the chunk's counts (na was counted per wave: every lane holds its wave's total)
  __syncthreads();
  if (lane == 0) sh.bins[t / WAVE] = (int)na;
  __syncthreads();
  if (t == 0) {
    int tot_a = 0;
    for (int i = 0; i < TS_WAVES; ++i) tot_a += sh.bins[i];
    int tot_c = 0;
    for (int i = 0; i < TS_G * TS_WAVES; ++i) tot_c += (int)sh.blk[i];
    meta[row].n_a[chunk] = tot_a;
    meta[row].n_c[chunk] = tot_c;
  }
}

struct OutShared {
  int hist[TK_BINS];
  int gt[TS_MAXCH], tie[TS_MAXCH], nc[TS_MAXCH], na[TS_MAXCH];
  int off[TS_MAXCH + 1];
  uint32_t blk[TS_G * TS_WAVES];
  int c0, above0, nvis, maxc;
  int sel_c, sel_above;
  uint32_t T;
  int room;
};

// One refinement pass's threshold bin, by wave 0 over the block-wide histogram of nbins bins (32 or 8 per lane):
// the bin holding the need-th largest key and the keys above it, into sh.sel_c / sh.sel_above.
__device__ __forceinline__ void wave0_find_bin(OutShared& sh, int nbins, int need) {
  const int lane = threadIdx.x & (WAVE - 1);
  constexpr int PER = TK_BINS / WAVE;
  const int per = nbins / WAVE;
  int hb[PER];
  const int4* h4 = reinterpret_cast<const int4*>(sh.hist);
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) {
    int4 v = make_int4(0, 0, 0, 0);
    if (4 * i < per) v = h4[(per / 4) * lane + i];
    hb[4 * i] = v.x;
    hb[4 * i + 1] = v.y;
    hb[4 * i + 2] = v.z;
    hb[4 * i + 3] = v.w;
  }
  int mine = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) mine += hb[i];
  int inc = mine;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int x = __shfl_down(inc, o, WAVE);
    if (lane + o < WAVE) inc += x;
  }
  int suf = inc - mine;
  int found = -1, above = 0;
  if (suf < need && suf + mine >= need) {
#pragma unroll
    for (int i = PER - 1; i >= 0; --i) {
      if (found < 0 && i < per) {
        if (suf + hb[i] >= need) {
          found = per * lane + i;
          above = suf;
        } else {
          suf += hb[i];
        }
      }
    }
  }
  const uint64_t who = __ballot(found >= 0);
  if (who) {
    const int src = (int)__builtin_ctzll(who);
    if (lane == src) {
      sh.sel_c = found;
      sh.sel_above = above;
    }
  } else if (lane == 0) {  // counts that do not match (a workspace that was not zero): stay in range
    sh.sel_c = 0;
    sh.sel_above = 0;
  }
}

__global__ __launch_bounds__(TS_THREADS) void topk_output_kernel(const float* __restrict__ scores, int stride,
                                                                 const int* __restrict__ len, int len_div,
                                                                 int len_mul, int keep, int vis_only, int nchunks,
                                                                 int* __restrict__ hist,
                                                                 const RowMeta* __restrict__ meta,
                                                                 const uint32_t* __restrict__ ckey,
                                                                 int* __restrict__ idx_out, int* __restrict__ cnt_out) {
  __shared__ OutShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  const int L = level_len(len, row, len_div, len_mul, stride);
  const int base = chunk * TS_CHUNK;
  // the row's meta in one round of loads (wave 0: lanes 0 .. 15 the chunk counts), counts clamped into range
  if (wave == 0) {
    int x = 0, y = 0;
    if (lane < TS_MAXCH && lane < nchunks) {
      x = meta[row].n_c[lane];
      y = meta[row].n_a[lane];
      x = x < 0 ? 0 : (x > TS_CHUNK ? TS_CHUNK : x);
      y = y < 0 ? 0 : (y > TS_CHUNK ? TS_CHUNK : y);
    }
    int inc = x;  // prefix of the candidate counts (lanes 0 .. 15)
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      const int u = __shfl_up(inc, o, WAVE);
      if (lane >= o) inc += u;
    }
    int mx = x;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) mx = max(mx, __shfl_xor(mx, o, WAVE));
    if (lane < TS_MAXCH) {
      sh.nc[lane] = x;
      sh.na[lane] = y;
      sh.off[lane] = inc - x;
      sh.gt[lane] = 0;
      sh.tie[lane] = 0;
    }
    if (lane == TS_MAXCH) sh.off[TS_MAXCH] = __shfl(inc, TS_MAXCH - 1, WAVE);
    if (lane == 0) {
      sh.c0 = meta[row].c0;
      sh.above0 = meta[row].above0;
      sh.nvis = meta[row].nvis;
      sh.maxc = mx;
    }
  }
  uint32_t key[TS_G][4];
  load_chunk_keys(scores + (size_t)row * stride, L, base, (stride & 3) == 0, vis_only, key);
  // leave the row's histogram zero for the next call (each chunk clears its share; every topk_chunk_kernel
  // workgroup has read it)
  int* hrow = hist + (size_t)row * TK_HBINS;
  for (int i = chunk * TS_THREADS + t; i < TK_HBINS; i += nchunks * TS_THREADS) hrow[i] = 0;
  __syncthreads();
  const int c0 = sh.c0, nvis = sh.nvis;
  uint32_t T = 0;
  int room = 0;
  if (c0 >= 0 && nvis > keep) {
    const uint32_t* crow = ckey + (size_t)row * TS_MAXCH * TS_CHUNK;
    uint32_t lo = (uint32_t)c0 << TK_HSHIFT;
    int need = keep - sh.above0;
    if (sh.maxc <= TS_THREADS) {
      // fast path: thread t holds the t-th candidate of every chunk (one round of 16 independent loads)
      uint32_t v[TS_MAXCH];
#pragma unroll
      for (int j = 0; j < TS_MAXCH; ++j) v[j] = (j < nchunks && t < sh.nc[j]) ? crow[j * TS_CHUNK + t] : 0u;
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
        constexpr int SB = TK_HSHIFT - TK_BITS;
        const int nb = pass == 0 ? TK_BINS : (1 << SB);
        for (int i = t; i < nb; i += TS_THREADS) sh.hist[i] = 0;
        __syncthreads();
        const uint32_t width = pass == 0 ? (1u << TK_HSHIFT) : (1u << SB);
#pragma unroll
        for (int j = 0; j < TS_MAXCH; ++j) {
          const uint32_t d = v[j] - lo;
          if (v[j] != 0u && d < width) atomicAdd(&sh.hist[pass == 0 ? (d >> SB) : d], 1);
        }
        __syncthreads();
        if (wave == 0) wave0_find_bin(sh, nb, need);
        __syncthreads();
        lo += (uint32_t)sh.sel_c << (pass == 0 ? SB : 0);
        need -= sh.sel_above;
        __syncthreads();
      }
      T = lo;
      room = need;
      // per chunk: candidates above T and tied at T (ballots, one add per wave and chunk)
#pragma unroll
      for (int j = 0; j < TS_MAXCH; ++j) {
        const uint64_t g = __ballot(v[j] != 0u && v[j] > T);
        const uint64_t q = __ballot(v[j] != 0u && v[j] == T);
        if (lane == 0 && (g | q)) {
          atomicAdd(&sh.gt[j], __popcll(g));
          atomicAdd(&sh.tie[j], __popcll(q));
        }
      }
      __syncthreads();
    } else {
      // many keys in one 12-bit bin (ties): the same passes over the lists in global memory
      for (int pass = 0; pass < 2; ++pass) {
        constexpr int SB = TK_HSHIFT - TK_BITS;
        const int nb = pass == 0 ? TK_BINS : (1 << SB);
        for (int i = t; i < nb; i += TS_THREADS) sh.hist[i] = 0;
        __syncthreads();
        const uint32_t width = pass == 0 ? (1u << TK_HSHIFT) : (1u << SB);
        for (int j = 0; j < nchunks; ++j)
          for (int i = t; i < sh.nc[j]; i += TS_THREADS) {
            const uint32_t k = crow[j * TS_CHUNK + i];
            const uint32_t d = k - lo;
            if (d < width) atomicAdd(&sh.hist[pass == 0 ? (d >> SB) : d], 1);
          }
        __syncthreads();
        if (wave == 0) wave0_find_bin(sh, nb, need);
        __syncthreads();
        lo += (uint32_t)sh.sel_c << (pass == 0 ? SB : 0);
        need -= sh.sel_above;
        __syncthreads();
      }
      T = lo;
      room = need;
      for (int j = 0; j < nchunks; ++j)
        for (int i = t; i < sh.nc[j]; i += TS_THREADS) {
          const uint32_t k = crow[j * TS_CHUNK + i];
          if (k > T) atomicAdd(&sh.gt[j], 1);
          if (k == T) atomicAdd(&sh.tie[j], 1);
        }
      __syncthreads();
    }
  }
  // this chunk's output base and the ties it may take
  int out_base = 0, ties_before = 0;
  for (int j = 0; j < chunk && j < nchunks; ++j) {
    const int na = sh.na[j];
    int take = room - ties_before;
    take = take < 0 ? 0 : (take > sh.tie[j] ? sh.tie[j] : take);
    out_base += na + sh.gt[j] + take;
    ties_before += sh.tie[j];
  }
  int room_here = room - ties_before;
  room_here = room_here < 0 ? 0 : room_here;

  // ordered output of the chunk: above T, and the first room_here keys equal to T
  const uint64_t below = lanes_below();
  uint64_t am[TS_G][4], tm[TS_G][4];
  uint32_t cnt[TS_G];
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    uint32_t na = 0, nt = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      am[e][c] = __ballot(key[e][c] > T);
      tm[e][c] = __ballot(T != 0 && key[e][c] == T);
      na += __popcll(am[e][c]);
      nt += __popcll(tm[e][c]);
    }
    cnt[e] = (na << 16) | nt;
  }
  uint32_t bb[TS_G];
  block_bases(cnt, sh.blk, bb);
  const int cnt_row = nvis < 0 ? 0 : (nvis < keep ? nvis : keep);
  int* orow = idx_out + (size_t)row * keep;
#pragma unroll
  for (int e = 0; e < TS_G; ++e) {
    int a_before = (int)(bb[e] >> 16), t_before = (int)(bb[e] & 0xffffu);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      a_before += __popcll(am[e][c] & below);
      t_before += __popcll(tm[e][c] & below);
    }
    const int p0 = base + 4 * (TS_THREADS * e + t);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool a = (am[e][c] >> lane) & 1ull;
      const bool ti = (tm[e][c] >> lane) & 1ull;
      const bool sel = a || (ti && t_before < room_here);
      const int o = out_base + a_before + (t_before < room_here ? t_before : room_here);
      if (sel && (unsigned)o < (unsigned)keep) orow[o] = p0 + c;  // in range whatever the counts
      a_before += a;
      t_before += ti;
    }
  }
  if (chunk == 0) {
    for (int i = cnt_row + t; i < keep; i += TS_THREADS) orow[i] = 0;
    if (t == 0) cnt_out[row] = cnt_row;
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

__global__ void topk_mask_fill_kernel(float* __restrict__ mask, int P) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < P) mask[(size_t)row * P + i] = NEG_INF;
}

__global__ void topk_mask_scatter_kernel(const int* __restrict__ idx, const int* __restrict__ cnt,
                                         float* __restrict__ mask, int keep, int P) {
  const int row = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < keep && k < cnt[row]) {
    const int p = idx[(size_t)row * keep + k];
    if ((unsigned)p < (unsigned)P) mask[(size_t)row * P + p] = 0.0f;
  }
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

// One workgroup per row up to TOPK_FLAT_MAX scores; longer rows are selected in two levels, recursively.
constexpr int TOPK_FLAT_MAX = 32 * TK_THREADS;
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
static bool topk_plan(long n, int keep, size_t* ws) {
  if (n <= TOPK_FLAT_MAX) {
    if (ws) *ws = 0;
    return true;
  }
  if (keep > TOPK_LONG_KEEP_MAX) return false;
  const int sub = topk_sub_block(n, keep);
  const long nb = (n + sub - 1) / sub, nc = (long)keep * sub;
  // level 1 (the sub-block maxima) runs flat; level 2 (the candidates) may split again
  if (nb > TOPK_FLAT_MAX || nc >= n) return false;
  if (!topk_plan(nc, keep, nullptr)) return false;
  if (ws) *ws = 0;
  return true;
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

size_t topk_hist_bytes(int B) { return up256((size_t)B * TK_HBINS * 4); }

// The flat selection's meta and candidate lists (after the histograms).
static size_t topk_flat_bytes(int B) {
  return up256((size_t)B * sizeof(RowMeta)) + up256((size_t)B * TS_MAXCH * TS_CHUNK * 4);
}

size_t topk_workspace_bytes(int B, int max_len, int keep) {
  return topk_hist_bytes(B) + topk_flat_bytes(B) + topk_level_bytes(B, max_len, keep);
}

bool topk_supported(int max_len, int keep, int vis_only) {
  if (keep < 1) return false;
  if (max_len <= TOPK_FLAT_MAX) return true;
  return vis_only && topk_plan(max_len, keep, nullptr);
}

// The flat selection's buffers inside the top-k workspace: the first-level histograms [B, 4096] (zero between calls),
// then the per-row meta and the candidate lists.
struct TopkBuffers {
  int* hist;
  RowMeta* meta;
  uint32_t* ckey;
};

static hipError_t launch_topk_level(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                    int max_len, int keep, int vis_only, int* idx, int* cnt, const TopkBuffers& tb,
                                    bool hist_ready, int B, hipStream_t s) {
  if (max_len > TS_MAXCH * TS_CHUNK) return hipErrorInvalidValue;
  const int nch = (max_len + TS_CHUNK - 1) / TS_CHUNK < 1 ? 1 : (max_len + TS_CHUNK - 1) / TS_CHUNK;
  if (!hist_ready) {
    launch("topk_hist_kernel", topk_hist_kernel, dim3(nch, B), dim3(TKH_THREADS), s, scores, stride, len, len_div, len_mul,
                       vis_only, tb.hist);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  launch("topk_chunk_kernel", topk_chunk_kernel, dim3(nch, B), dim3(TS_THREADS), s, scores, stride, len, len_div, len_mul,
                     keep, vis_only, tb.hist, tb.meta, tb.ckey);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch("topk_output_kernel", topk_output_kernel, dim3(nch, B), dim3(TS_THREADS), s, scores, stride, len, len_div, len_mul,
                     keep, vis_only, nch, tb.hist, tb.meta, tb.ckey, idx, cnt);
  return hipGetLastError();
}

// Selection over rows of `stride` scores whose lengths are len[row] (len_div / len_mul as in topk_kernel), n an upper
// bound of the lengths.
static hipError_t topk_rows(const float* scores, int stride, const int* len, int len_div, int len_mul, long n,
                            int keep, int vis_only, int* idx, int* cnt, const TopkBuffers& tb, bool hist_ready,
                            char* ws, int B, hipStream_t s) {
  if (n <= TOPK_FLAT_MAX)
    return launch_topk_level(scores, stride, len, len_div, len_mul, (int)n, keep, vis_only, idx, cnt, tb,
                             hist_ready, B, s);
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
  launch("block_max_kernel", block_max_kernel, dim3((nb + 255) / 256, B), dim3(256), s, scores, stride, len, sub, nb, bm);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // level 1: the top-keep sub-blocks (ceil(len / sub) maxima per row)
  if (nb > TOPK_FLAT_MAX) return hipErrorInvalidValue;  // excluded by topk_plan
  e = launch_topk_level(bm, nb, len, sub, 1, nb, keep, vis_only, bidx, bcnt, tb, false, B, s);
  if (e != hipSuccess) return e;
  launch("gather_blocks_kernel", gather_blocks_kernel, dim3((nc + 255) / 256, B), dim3(256), s, scores, stride, len, sub, bidx,
                     bcnt, keep, cand);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // level 2: the top-keep of the selected sub-blocks' scores in position order (NEG_INF past their count)
  e = topk_rows(cand, nc, nullptr, 1, 1, nc, keep, vis_only, idx, cnt, tb, false, ws, B, s);
  if (e != hipSuccess) return e;
  launch("map_blocks_kernel", map_blocks_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, bidx, sub, keep);
  return hipGetLastError();
}

// ws: topk_workspace_bytes(B, max_len, keep) bytes whose histogram region is zero; hist_ready: the histogram of the
// rows is already accumulated there (by the indexer), so the first level skips its histogram kernel.
hipError_t launch_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                       int max_len, int keep, int vis_only, bool hist_ready, hipStream_t s) {
  char* p = static_cast<char*>(ws);
  if (hist_ready && max_len > TOPK_FLAT_MAX) return hipErrorInvalidValue;  // the indexer histograms flat rows only
  TopkBuffers tb;
  tb.hist = reinterpret_cast<int*>(p);
  p += topk_hist_bytes(B);
  tb.meta = reinterpret_cast<RowMeta*>(p);
  p += up256((size_t)B * sizeof(RowMeta));
  tb.ckey = reinterpret_cast<uint32_t*>(p);
  p += up256((size_t)B * TS_MAXCH * TS_CHUNK * 4);
  return topk_rows(scores, stride, len, 1, 1, max_len, keep, vis_only, idx, cnt, tb, hist_ready, p, B, s);
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

hipError_t launch_topk_mask(const int* idx, const int* cnt, float* mask, int B, int keep, int P, hipStream_t s) {
  launch("topk_mask_fill_kernel", topk_mask_fill_kernel, dim3((P + 255) / 256, B), dim3(256), s, mask, P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch("topk_mask_scatter_kernel", topk_mask_scatter_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, mask, keep,
                     P);
  return hipGetLastError();
}

}  // namespace dsa
