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
constexpr int TK_BINS = 2048;
constexpr int TK_BITS = 11;

struct TopkShared {
  int hist[TK_BINS];
  int red_i[TK_WAVES];
  uint32_t red_u[2][TK_WAVES];
  int scan_tot[TK_WAVES];
  int sel_bin;
  int sel_above;
};

// Block-wide exclusive prefix sum of one int per thread (position order = thread order); returns the prefix and
// writes the total to *total.
__device__ __forceinline__ int block_excl_scan(int v, TopkShared& sh, int* total) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  const int inc = wave_incl_scan(v);
  if (lane == WAVE - 1) sh.scan_tot[wave] = inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) {
    const int t = sh.scan_tot[i];
    before += i < wave ? t : 0;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

__device__ __forceinline__ int block_sum(int v, TopkShared& sh) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  v = wave_sum(v);
  if (lane == 0) sh.red_i[wave] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) t += sh.red_i[i];
  __syncthreads();
  return t;
}

__device__ __forceinline__ void block_minmax(uint32_t& mn, uint32_t& mx, TopkShared& sh) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  mn = wave_min_u32(mn);
  mx = wave_max_u32(mx);
  if (lane == 0) {
    sh.red_u[0][wave] = mn;
    sh.red_u[1][wave] = mx;
  }
  __syncthreads();
  mn = 0xffffffffu;
  mx = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) {
    mn = min(mn, sh.red_u[0][i]);
    mx = max(mx, sh.red_u[1][i]);
  }
  __syncthreads();
}

// Given the histogram of the keys inside the interval, finds the bin c holding the need-th largest key
// (suffix(c) >= need > suffix(c + 1)); returns c and sets *above_in = suffix(c + 1).
__device__ __forceinline__ int find_bin(int need, int* above_in, TopkShared& sh) {
  const int t = threadIdx.x;
  // thread t owns bins 2t, 2t + 1; suffix order: thread TK_THREADS - 1 first.
  const int b0 = 2 * t, b1 = 2 * t + 1;
  const int h0 = sh.hist[b0], h1 = sh.hist[b1];
  // exclusive suffix sum over threads: scan over reversed thread order
  const int rt = TK_THREADS - 1 - t;
  const int wave = rt / WAVE, lane = rt & (WAVE - 1);
  const int v = h0 + h1;
  // wave scan in reversed lane order: use the reversed id's lane within its wave
  int inc = v;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    // lanes of the reversed order: rt's wave holds threads with the same t / 64 (reversed lanes)
    int tt = __shfl_down(inc, o, WAVE);  // thread t + o has reversed lane - o
    if (lane >= o) inc += tt;
  }
  __syncthreads();  // hist reads done before scan_tot is reused below
  if (lane == WAVE - 1) sh.scan_tot[wave] = inc;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int i = 0; i < TK_WAVES; ++i) before += i < wave ? sh.scan_tot[i] : 0;
  const int suf_after = before + inc - v;  // keys in bins above b1
  // bin b1 first (higher), then b0
  if (suf_after < need && suf_after + h1 >= need) {
    sh.sel_bin = b1;
    sh.sel_above = suf_after;
  } else if (suf_after + h1 < need && suf_after + h1 + h0 >= need) {
    sh.sel_bin = b0;
    sh.sel_above = suf_after + h1;
  }
  __syncthreads();
  const int c = sh.sel_bin;
  *above_in = sh.sel_above;
  __syncthreads();
  return c;
}

__device__ __forceinline__ int bit_length(uint32_t x) { return x ? 32 - __clz(x) : 0; }

// Row r's output positions: map_blocks (two-level) turns a candidate position p into map[p / sub] * sub + p % sub.
template <int E>
__global__ __launch_bounds__(TK_THREADS) void topk_kernel(const float* __restrict__ scores, int stride,
                                                          const int* __restrict__ len, int len_div, int len_mul,
                                                          int keep, int vis_only, const int* __restrict__ map_blocks,
                                                          int map_sub, int map_stride, int* __restrict__ idx_out,
                                                          int* __restrict__ cnt_out) {
  __shared__ TopkShared sh;
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  int L = stride;
  if (len) {
    // the row length in elements of this level: len[row] for a flat row; ceil(len / len_div) for block maxima;
    // len[row] * len_mul for a candidate row of len[row] sub-blocks
    long l = len[row];
    l = l < 0 ? 0 : l;
    if (len_div > 1) l = (l + len_div - 1) / len_div;
    if (len_mul > 1) l *= len_mul;
    L = (int)(l < stride ? l : stride);
  }
  const float* srow = scores + (size_t)row * stride;
  const int p0 = t * E;

  uint32_t key[E];
  const bool vec = ((stride & 3) == 0) && ((E & 3) == 0);
  if (vec && p0 + E <= L) {
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(srow + p0 + e);
      key[e + 0] = (!vis_only || v.x > VISIBLE) ? order_key(v.x) : 0u;
      key[e + 1] = (!vis_only || v.y > VISIBLE) ? order_key(v.y) : 0u;
      key[e + 2] = (!vis_only || v.z > VISIBLE) ? order_key(v.z) : 0u;
      key[e + 3] = (!vis_only || v.w > VISIBLE) ? order_key(v.w) : 0u;
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int p = p0 + e;
      uint32_t k = 0;
      if (p < L) {
        const float v = srow[p];
        k = (!vis_only || v > VISIBLE) ? order_key(v) : 0u;
      }
      key[e] = k;
    }
  }

  // selectable count and key range
  int nv = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t k = key[e];
    nv += k != 0;
    if (k) {
      kmin = min(kmin, k);
      kmax = max(kmax, k);
    }
  }
  const int nvis = block_sum(nv, sh);
  block_minmax(kmin, kmax, sh);

  uint32_t T = 0;  // select key > T, plus `room` keys == T by position
  int room = 0;
  if (nvis > keep) {
    uint32_t lo = kmin, hi = kmax;
    int need = keep;
    bool first = true;
    while (lo != hi) {
      for (int i = t; i < TK_BINS; i += TK_THREADS) sh.hist[i] = 0;
      __syncthreads();
      const float flo = key_to_float(lo), fhi = key_to_float(hi);
      const float span = fhi - flo;
      const bool linear = first && isfinite(flo) && isfinite(fhi) && isfinite(span) && span > 0.0f;
      const float inv = linear ? (float)TK_BINS / span : 0.0f;
      const int sh_bits = max(0, bit_length(hi - lo) - TK_BITS);
      auto bin_of = [&](uint32_t k) -> int {
        if (linear) {
          const float f = key_to_float(k);
          int c = (int)((f - flo) * inv);
          return c < 0 ? 0 : (c >= TK_BINS ? TK_BINS - 1 : c);
        }
        return (int)((k - lo) >> sh_bits);
      };
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const uint32_t k = key[e];
        if (k >= lo && k <= hi) atomicAdd(&sh.hist[bin_of(k)], 1);
      }
      __syncthreads();
      int above_in = 0;
      const int c = find_bin(need, &above_in, sh);
      need -= above_in;
      if (linear) {
        // the keys of bin c form a key interval; its bounds are the min / max key that falls into it
        uint32_t nlo = 0xffffffffu, nhi = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint32_t k = key[e];
          if (k >= lo && k <= hi && bin_of(k) == c) {
            nlo = min(nlo, k);
            nhi = max(nhi, k);
          }
        }
        block_minmax(nlo, nhi, sh);
        lo = nlo;
        hi = nhi;
      } else {
        const uint32_t nlo = lo + ((uint32_t)c << sh_bits);
        const uint32_t width = sh_bits >= 32 ? 0xffffffffu : ((1u << sh_bits) - 1u);
        const uint32_t nhi = (hi - nlo > width) ? nlo + width : hi;
        lo = nlo;
        hi = nhi;
      }
      first = false;
    }
    T = lo;
    room = need;
  }

  // tied keys before this thread's positions (position order = thread order, then e)
  int na = 0, nt = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    na += key[e] > T;
    nt += (T != 0) && (key[e] == T);
  }
  int tot = 0;
  const int tie_before = block_excl_scan(nt, sh, &tot);
  int take = room - tie_before;  // ties this thread may take
  take = take < 0 ? 0 : (take > nt ? nt : take);
  const int ns = na + take;
  const int out_before = block_excl_scan(ns, sh, &tot);
  const int cnt = nvis < keep ? nvis : keep;
  int* orow = idx_out + (size_t)row * keep;
  int o = out_before, taken = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t k = key[e];
    bool sel = k > T;
    if (!sel && T != 0 && k == T && taken < take) {
      sel = true;
      ++taken;
    }
    if (sel) {
      int p = p0 + e;
      if (map_blocks) p = map_blocks[(size_t)row * map_stride + p / map_sub] * map_sub + p % map_sub;
      orow[o++] = p;
    }
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

static size_t topk_ws_bytes(int B, long n, int keep) {
  if (n <= TOPK_FLAT_MAX) return 0;
  const int sub = topk_sub_block(n, keep);
  const long nb = (n + sub - 1) / sub, nc = (long)keep * sub;
  const size_t own = up256((size_t)B * nb * 4) + up256((size_t)B * keep * 4) + up256((size_t)B * 4) +
                     up256((size_t)B * nc * 4);
  const size_t a = topk_ws_bytes(B, nb, keep), c = topk_ws_bytes(B, nc, keep);
  return own + (a > c ? a : c);
}

size_t topk_workspace_bytes(int B, int max_len, int keep) { return topk_ws_bytes(B, max_len, keep); }

bool topk_supported(int max_len, int keep, int vis_only) {
  if (keep < 1) return false;
  if (max_len <= TOPK_FLAT_MAX) return true;
  return vis_only && topk_plan(max_len, keep, nullptr);
}

static hipError_t launch_topk_level(const float* scores, int stride, const int* len, int len_div, int len_mul,
                                    int max_len, int keep, int vis_only, int* idx, int* cnt, int B, hipStream_t s) {
  const int E = topk_elems(max_len);
#define TK_CASE(EV)                                                                                             \
  case EV:                                                                                                      \
    hipLaunchKernelGGL(topk_kernel<EV>, dim3(B), dim3(TK_THREADS), 0, s, scores, stride, len, len_div, len_mul, \
                       keep, vis_only, nullptr, 1, 0, idx, cnt);                                                \
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
                            int keep, int vis_only, int* idx, int* cnt, char* ws, int B, hipStream_t s) {
  if (n <= TOPK_FLAT_MAX)
    return launch_topk_level(scores, stride, len, len_div, len_mul, (int)n, keep, vis_only, idx, cnt, B, s);
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
  e = launch_topk_level(bm, nb, len, sub, 1, nb, keep, vis_only, bidx, bcnt, B, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gather_blocks_kernel, dim3((nc + 255) / 256, B), dim3(256), 0, s, scores, stride, len, sub, bidx,
                     bcnt, keep, cand);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // level 2: the top-keep of the selected sub-blocks' scores in position order (NEG_INF past their count)
  e = topk_rows(cand, nc, nullptr, 1, 1, nc, keep, vis_only, idx, cnt, ws, B, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(map_blocks_kernel, dim3((keep + 255) / 256, B), dim3(256), 0, s, idx, cnt, bidx, sub, keep);
  return hipGetLastError();
}

hipError_t launch_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                       int max_len, int keep, int vis_only, hipStream_t s) {
  return topk_rows(scores, stride, len, 1, 1, max_len, keep, vis_only, idx, cnt, static_cast<char*>(ws), B, s);
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
