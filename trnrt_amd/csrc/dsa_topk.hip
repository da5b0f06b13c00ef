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

// The selection of one row (E scores per thread, positions t E .. t E + E - 1), given the row's first-level
// histogram: the threshold's 12-bit bin from the histogram, the threshold inside it by two passes over the low key
// bits (only keys inside the bin count), then the ordered output. Re-zeroes the histogram.
template <int E>
__global__ __launch_bounds__(TK_THREADS) void topk_select_kernel(const float* __restrict__ scores, int stride,
                                                                 const int* __restrict__ len, int len_div,
                                                                 int len_mul, int keep, int vis_only,
                                                                 int* __restrict__ hist, int* __restrict__ idx_out,
                                                                 int* __restrict__ cnt_out) {
  __shared__ TopkShared sh;
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const int L = level_len(len, row, len_div, len_mul, stride);
  const float* srow = scores + (size_t)row * stride;
  const int p0 = t * E;

  // the row's histogram (4 bins per thread) and keys
  int* hrow = hist + (size_t)row * TK_HBINS;
  const int4 hv = *reinterpret_cast<const int4*>(hrow + 4 * t);
  uint32_t key[E];
  if (((stride & 3) == 0) && ((E & 3) == 0) && p0 + E <= L) {
    float4 raw[E / 4];
#pragma unroll
    for (int e = 0; e < E / 4; ++e) raw[e] = *reinterpret_cast<const float4*>(srow + p0 + 4 * e);
#pragma unroll
    for (int e = 0; e < E / 4; ++e) {
      key[4 * e + 0] = select_key(raw[e].x, vis_only);
      key[4 * e + 1] = select_key(raw[e].y, vis_only);
      key[4 * e + 2] = select_key(raw[e].z, vis_only);
      key[4 * e + 3] = select_key(raw[e].w, vis_only);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) key[e] = (p0 + e < L) ? select_key(srow[p0 + e], vis_only) : 0u;
  }

  // threshold bin among this thread's 4 (bins 4t .. 4t + 3, higher bins first). The defaults keep every index in
  // range should the histogram not match the scores (a workspace that was not zero): the selection is then wrong but
  // every write stays inside its buffer.
  if (t == 0) {
    sh.sel_bin = 0;
    sh.sel_above = 0;
  }
  int nvis = 0;
  const int hsum = hv.x + hv.y + hv.z + hv.w;
  const int above4 = block_excl_suffix(hsum, sh, &nvis);  // keys in bins above 4t + 3
  *reinterpret_cast<int4*>(hrow + 4 * t) = make_int4(0, 0, 0, 0);  // leave the histogram zero for the next call
  uint32_t T = 0;  // select key > T, plus the first `room` keys == T by position
  int room = 0;
  if (nvis > keep) {
    {
      const int hb[4] = {hv.x, hv.y, hv.z, hv.w};
      int suf = above4;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (suf < keep && suf + hb[i] >= keep) {
          sh.sel_bin = 4 * t + i;
          sh.sel_above = suf;
        }
        suf += hb[i];
      }
    }
    __syncthreads();
    const int c0 = sh.sel_bin & (TK_HBINS - 1);
    int need = keep - sh.sel_above;
    uint32_t lo = (uint32_t)c0 << TK_HSHIFT, hi = lo | ((1u << TK_HSHIFT) - 1u);
    while (lo != hi) {
      for (int i = t; i < TK_BINS; i += TK_THREADS) sh.hist[i] = 0;
      __syncthreads();
      const int sb = max(0, bit_length(hi - lo) - TK_BITS);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const uint32_t k = key[e];
        if (k >= lo && k <= hi) atomicAdd(&sh.hist[(k - lo) >> sb], 1);
      }
      __syncthreads();
      // the bin of the need-th largest key inside [lo, hi] (2 bins per thread)
      const int h0 = sh.hist[2 * t], h1 = sh.hist[2 * t + 1];
      if (t == 0) {
        sh.sel_bin = 0;
        sh.sel_above = 0;
      }
      int tot = 0;
      const int suf = block_excl_suffix(h0 + h1, sh, &tot);
      if (suf < need && suf + h1 >= need) {
        sh.sel_bin = 2 * t + 1;
        sh.sel_above = suf;
      } else if (suf + h1 < need && suf + h1 + h0 >= need) {
        sh.sel_bin = 2 * t;
        sh.sel_above = suf + h1;
      }
      __syncthreads();
      const int c = sh.sel_bin & (TK_BINS - 1);
      need -= sh.sel_above;
      __syncthreads();
      const uint32_t nlo = lo + ((uint32_t)c << sb);
      const uint32_t width = (1u << sb) - 1u;
      hi = (hi - nlo > width) ? nlo + width : hi;
      lo = nlo;
    }
    T = lo;
    room = need;
  }

  // ordered output: one scan of the packed (above, tied) counts; the selected before a position are the keys above
  // T before it plus min(room, ties before it)
  uint32_t na = 0, nt = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    na += key[e] > T;
    nt += (T != 0) && (key[e] == T);
  }
  uint32_t tot = 0;
  const uint32_t before = block_excl_scan((na << 16) | nt, sh, &tot);
  const int above_before = (int)(before >> 16), tie_before = (int)(before & 0xffffu);
  int take = room - tie_before;
  take = take < 0 ? 0 : (take > (int)nt ? (int)nt : take);
  int o = above_before + (tie_before < room ? tie_before : room);
  const int cnt = nvis < 0 ? 0 : (nvis < keep ? nvis : keep);
  int* orow = idx_out + (size_t)row * keep;
  int taken = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t k = key[e];
    const bool tie = T != 0 && k == T && taken < take;
    taken += tie;
    if ((k > T || tie) && (unsigned)o < (unsigned)keep) orow[o++] = p0 + e;  // in range whatever the counts
  }
  for (int i = cnt + t; i < keep; i += TK_THREADS) orow[i] = 0;
  if (t == 0) cnt_out[row] = cnt;
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

static int topk_elems(int n) {
  for (int e = 4; e <= 32; e *= 2)
    if ((long)e * TK_THREADS >= n) return e;
  return 0;
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

size_t topk_workspace_bytes(int B, int max_len, int keep) {
  return topk_hist_bytes(B) + topk_level_bytes(B, max_len, keep);
}

bool topk_supported(int max_len, int keep, int vis_only) {
  if (keep < 1) return false;
  if (max_len <= TOPK_FLAT_MAX) return true;
  return vis_only && topk_plan(max_len, keep, nullptr);
}

static hipError_t launch_topk_level(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                    int max_len, int keep, int vis_only, int* idx, int* cnt, int* hist, bool hist_ready,
                                    int B, hipStream_t s) {
  const int E = topk_elems(max_len);
  if (!E) return hipErrorInvalidValue;
  if (!hist_ready) {
    hipLaunchKernelGGL(topk_hist_kernel, dim3((max_len + TKH_CHUNK - 1) / TKH_CHUNK, B), dim3(TKH_THREADS), 0, s,
                       scores, stride, len, len_div, len_mul, vis_only, hist);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
#define TK_CASE(EV)                                                                                             \
  case EV:                                                                                                      \
    hipLaunchKernelGGL(topk_select_kernel<EV>, dim3(B), dim3(TK_THREADS), 0, s, scores, stride, len, len_div,   \
                       len_mul, keep, vis_only, hist, idx, cnt);                                                \
    break;
  switch (E) {
    TK_CASE(4)
    TK_CASE(8)
    TK_CASE(16)
    TK_CASE(32)
    default:
      return hipErrorInvalidValue;
  }
#undef TK_CASE
  return hipGetLastError();
}

// Selection over rows of `stride` scores whose lengths are len[row] (len_div / len_mul as in topk_kernel), n an upper
// bound of the lengths.
static hipError_t topk_rows(const float* scores, int stride, const int* len, int len_div, int len_mul, long n,
                            int keep, int vis_only, int* idx, int* cnt, int* hist, bool hist_ready, char* ws, int B,
                            hipStream_t s) {
  if (n <= TOPK_FLAT_MAX)
    return launch_topk_level(scores, stride, len, len_div, len_mul, (int)n, keep, vis_only, idx, cnt, hist,
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
  hipLaunchKernelGGL(block_max_kernel, dim3((nb + 255) / 256, B), dim3(256), 0, s, scores, stride, len, sub, nb, bm);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // level 1: the top-keep sub-blocks (ceil(len / sub) maxima per row)
  if (nb > TOPK_FLAT_MAX) return hipErrorInvalidValue;  // excluded by topk_plan
  e = launch_topk_level(bm, nb, len, sub, 1, nb, keep, vis_only, bidx, bcnt, hist, false, B, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gather_blocks_kernel, dim3((nc + 255) / 256, B), dim3(256), 0, s, scores, stride, len, sub, bidx,
                     bcnt, keep, cand);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // level 2: the top-keep of the selected sub-blocks' scores in position order (NEG_INF past their count)
  e = topk_rows(cand, nc, nullptr, 1, 1, nc, keep, vis_only, idx, cnt, hist, false, ws, B, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(map_blocks_kernel, dim3((keep + 255) / 256, B), dim3(256), 0, s, idx, cnt, bidx, sub, keep);
  return hipGetLastError();
}

// ws: topk_workspace_bytes(B, max_len, keep) bytes whose histogram region is zero; hist_ready: the histogram of the
// rows is already accumulated there (by the indexer), so the first level skips its histogram kernel.
hipError_t launch_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                       int max_len, int keep, int vis_only, bool hist_ready, hipStream_t s) {
  char* p = static_cast<char*>(ws);
  int* hist = reinterpret_cast<int*>(p);
  if (hist_ready && max_len > TOPK_FLAT_MAX) return hipErrorInvalidValue;  // the indexer histograms flat rows only
  return topk_rows(scores, stride, len, 1, 1, max_len, keep, vis_only, idx, cnt, hist, hist_ready,
                   p + topk_hist_bytes(B), B, s);
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
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, s, static_cast<uint4*>(p), n16);
  }
  return hipGetLastError();
}

hipError_t launch_topk_mask(const int* idx, const int* cnt, float* mask, int B, int keep, int P, hipStream_t s) {
  hipLaunchKernelGGL(topk_mask_fill_kernel, dim3((P + 255) / 256, B), dim3(256), 0, s, mask, P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(topk_mask_scatter_kernel, dim3((keep + 255) / 256, B), dim3(256), 0, s, idx, cnt, mask, keep,
                     P);
  return hipGetLastError();
}

}  // namespace dsa
