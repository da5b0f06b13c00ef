// Compaction kernels: a 0 / 1 mask's ones as ascending indices (trnrt/models/dsa_long.py:140-166 `compact`), and a
// slot list's visible tokens as one compacted token list per row, the gather list of the compacted slot attention
// (trnrt/kernels/dsa_slots_c.py:1-37: a row attends only the slots that hold a visible token).
//
// One workgroup of 256 threads per row walks the row in chunks of 2,048 entries, each thread 8 consecutive entries:
// a thread's ones as an 8-bit mask, their block-wide exclusive prefix (a DPP wave scan plus the 4 wave totals through
// LDS) and the running count before the chunk give each one its output index, written in order. The walk stops once
// keep ones are placed, so a row costs at most its leading entries.
#include "dsa_common.h"

namespace dsa {

constexpr int CP_THREADS = 256;
constexpr int CP_WAVES = CP_THREADS / WAVE;
constexpr int CP_PER = 8;  // entries per thread and chunk

// Block-wide exclusive prefix of v over the 256 threads, the total into *tot. scr: CP_WAVES ints of LDS; the call
// ends with a barrier, so scr may be written again right after.
__device__ __forceinline__ int cp_block_prefix(int v, int* scr, int* tot) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  const int incl = wave_incl_scan(v);
  if (lane == WAVE - 1) scr[wave] = incl;
  __syncthreads();
  int before = incl - v, t = 0;
#pragma unroll
  for (int w = 0; w < CP_WAVES; ++w) {
    const int x = scr[w];
    before += w < wave ? x : 0;
    t += x;
  }
  *tot = t;
  __syncthreads();
  return before;
}

// Row n of sel [N, M] (an entry counts as a one when above 0.5): the positions of its first keep ones, ascending, into
// idx [N, keep] (0 past the count) and the count min(ones, keep) into cnt [N].
__global__ __launch_bounds__(CP_THREADS) void compact_mask_kernel(const float* __restrict__ sel, int M, int keep,
                                                                   int64_t* __restrict__ idx,
                                                                   int64_t* __restrict__ cnt) {
  __shared__ int scr[CP_WAVES];
  const int n = blockIdx.x, tid = threadIdx.x;
  const float* row = sel + (size_t)n * M;
  int64_t* irow = idx + (size_t)n * keep;
  int base = 0;  // ones before the chunk (block-uniform)
  for (int c0 = 0; c0 < M && base < keep; c0 += CP_PER * CP_THREADS) {
    const int p0 = c0 + CP_PER * tid;
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < CP_PER; ++i)
      if (p0 + i < M && row[p0 + i] > 0.5f) bits |= 1u << i;
    int tot;
    int o = base + cp_block_prefix(__builtin_popcount(bits), scr, &tot);
    while (bits && o < keep) {
      const int i = __builtin_ctz(bits);
      bits &= bits - 1u;
      irow[o++] = p0 + i;
    }
    base += tot;
  }
  const int c = min(base, keep);
  for (int o = c + tid; o < keep; o += CP_THREADS) irow[o] = 0;
  if (tid == 0) cnt[n] = c;
}

// Row b of a slot list (rows [B, NS] pool rows of a cache viewed as [pools, kp rows], bias [B, NS, kp], a token
// visible when its bias is above NEG_INF / 2): the visible tokens' cache rows pool kp + t in slot order into
// tok [B, NS kp] and their count into tcnt [B]. A row with none lists pool row 0's kp tokens (the attention then
// weighs them uniformly: the empty entries of the compacted form are pool row 0 with no visible token). Pool rows
// outside [0, pools) read pool 0. Entries past the list are 0.
__global__ __launch_bounds__(CP_THREADS) void compact_slots_kernel(const int* __restrict__ rows,
                                                                    const float* __restrict__ bias, int NS, int kp,
                                                                    int pools, int* __restrict__ tok,
                                                                    int* __restrict__ tcnt) {
  __shared__ int scr[CP_WAVES];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int T = NS * kp;
  const float* brow = bias + (size_t)b * T;
  const int* rrow = rows + (size_t)b * NS;
  int* trow = tok + (size_t)b * T;
  int base = 0;
  for (int c0 = 0; c0 < T; c0 += CP_PER * CP_THREADS) {
    const int e0 = c0 + CP_PER * tid;
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < CP_PER; ++i)
      if (e0 + i < T && brow[e0 + i] > NEG_INF * 0.5f) bits |= 1u << i;
    int tot;
    int o = base + cp_block_prefix(__builtin_popcount(bits), scr, &tot);
    while (bits) {
      const int i = __builtin_ctz(bits);
      bits &= bits - 1u;
      const int e = e0 + i, s = e / kp;
      const int pr = rrow[s];
      trow[o++] = ((unsigned)pr < (unsigned)pools ? pr : 0) * kp + (e - s * kp);
    }
    base += tot;
  }
  for (int o = base + tid; o < T; o += CP_THREADS) trow[o] = base == 0 && o < kp ? o : 0;
  if (tid == 0) tcnt[b] = base;
}

// A selection (pools [N, keep] ascending, cnt [N], vals [N, keep]) in value order (trnrt/kernels/
// dsa_long_select.py:74-84, the "vorder" output): a row's live entries (k < cnt) by value descending, equal values by
// pool ascending, then pool 0 / NEG_INF. One workgroup per row sorts 64-bit keys (the value's order-preserving key,
// then the inverted entry index, so equal values keep the input's ascending pool order; dead entries key 0, last) by
// a bitonic network in LDS over the next power of two >= keep (at most VO_MAX), and gathers pools and values by the
// sorted indices (the values copied, not rebuilt from their keys).
constexpr int VO_MAX = 8192;
constexpr int VO_THREADS = 512;

__global__ __launch_bounds__(VO_THREADS) void value_order_kernel(const int64_t* __restrict__ pools,
                                                                  const int64_t* __restrict__ cnt,
                                                                  const float* __restrict__ vals, int keep, int np2,
                                                                  int64_t* __restrict__ out_pools,
                                                                  float* __restrict__ out_vals) {
  __shared__ uint64_t key[VO_MAX];
  const int n = blockIdx.x, tid = threadIdx.x;
  const int64_t c = cnt[n];
  const float* vr = vals + (size_t)n * keep;
  for (int k = tid; k < np2; k += VO_THREADS) {
    const bool live = k < keep && k < c;
    key[k] = live ? ((uint64_t)order_key(vr[k]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)k) : 0ull;
  }
  __syncthreads();
  // bitonic network, descending overall: pairs (i, i ^ j) with i < i ^ j, direction by bit `size` of i
  for (int size = 2; size <= np2; size <<= 1) {
    for (int j = size >> 1; j > 0; j >>= 1) {
      for (int t = tid; t < np2 / 2; t += VO_THREADS) {
        const int i = 2 * t - (t & (j - 1));  // the lower index of the t-th pair at distance j
        const int l = i + j;
        const uint64_t a = key[i], b = key[l];
        const bool desc = (i & size) == 0;
        if (desc ? a < b : a > b) {
          key[i] = b;
          key[l] = a;
        }
      }
      __syncthreads();
    }
  }
  const int64_t* pr = pools + (size_t)n * keep;
  for (int k = tid; k < keep; k += VO_THREADS) {
    const uint64_t kk = key[k];
    const bool live = kk != 0ull;
    const int src = (int)(0xFFFFFFFFu - (uint32_t)kk);
    out_pools[(size_t)n * keep + k] = live ? pr[src] : 0;
    out_vals[(size_t)n * keep + k] = live ? vr[src] : NEG_INF;
  }
}

hipError_t launch_value_order(const int64_t* pools, const int64_t* cnt, const float* vals, int N, int keep,
                              int64_t* out_pools, float* out_vals, hipStream_t s) {
  int np2 = 2;
  while (np2 < keep) np2 <<= 1;
  return launch("value_order_kernel", value_order_kernel, dim3(N), dim3(VO_THREADS), s, pools, cnt, vals, keep, np2,
                out_pools, out_vals);
}

hipError_t launch_compact_mask(const float* sel, int N, int M, int keep, int64_t* idx, int64_t* cnt, hipStream_t s) {
  return launch("compact_mask_kernel", compact_mask_kernel, dim3(N), dim3(CP_THREADS), s, sel, M, keep, idx, cnt);
}

hipError_t launch_compact_slots(const int* rows, const float* bias, int B, int NS, int kp, int pools, int* tok,
                                int* tcnt, hipStream_t s) {
  return launch("compact_slots_kernel", compact_slots_kernel, dim3(B), dim3(CP_THREADS), s, rows, bias, NS, kp, pools,
                tok, tcnt);
}

}  // namespace dsa
