// Sparse MLA decode attention for gfx950 over the selected tokens of a paged FP8 latent cache (the arithmetic of
// trnrt/kernels/dsa_decode.py:26-37 and trnrt/kernels/dsa_slots.py:48-65, absorbed MLA, with a 576-wide key of
// 512 latent + 64 rope columns and the first 512 columns as the value; per-token FP8 scales):
//
//   s[h, k] = scale * q[h, :] . K[k] + bias[k],  K[k] = kv_fp8[slot_k] * kv_scale[slot_k]
//   o[h, :] = sum_k softmax_k(s)[h, k] * K[k][:512],  lse[h] = max_k s + log sum_k exp(s - max)
//
// Work unit: one workgroup = one sequence, 16 query heads, one split of the selected slots (split-K), in chunks of
// 64 slots. Per chunk the 64 gathered rows are staged in LDS twice: token-major (e4m3 bytes, for the score product
// whose contraction runs over a row) and dim-major for the first 512 columns (for the value product, whose
// contraction runs over the tokens; an in-register 4x4 byte transpose through LDS). Both products run on
// v_mfma_f32_16x16x32_bf16 with e4m3 -> bf16 conversions in registers (exact).
//   - scores: S^T[token, head] = K . Q^T; wave w takes tokens 16w .. 16w + 15 of the chunk, all 16 heads, the 576
//     dims in 18 steps (dims permuted so a lane reads 144 contiguous bytes of its row; q uses the same permutation);
//   - online softmax in fp32 with the chunk maximum shared through LDS (every wave applies the same rescale);
//   - value: O[head, dim] += P . V with P = exp(s - m) * kv_scale rounded to bf16 (the dequantisation of the value
//     folded into the weight), wave w takes dims 128w .. 128w + 127.
// With one split the workgroup writes bf16 o and lse; with several it writes fp32 partial o (normalised) with its
// running max and sum, and a combine kernel merges them by log-sum-exp (trnrt/models/mla.py:853-856, 1152-1160).
#include "dsa_common.h"

namespace dsa {

constexpr int ATT_DQK = 576;
constexpr int ATT_DV = 512;
constexpr int ATT_HPW = 16;       // heads per workgroup
constexpr int ATT_CH = 64;        // slots per chunk
constexpr int ATT_THREADS = 256;  // 4 waves
constexpr int ATT_KROW = ATT_DQK + 16;  // token-major row stride (bytes)
constexpr int ATT_VROW = ATT_CH + 4;    // dim-major row stride (bytes)
constexpr int ATT_PROW = ATT_CH + 4;    // P row stride (bf16 elements)

struct AttShared {
  uint8_t kt[ATT_CH * ATT_KROW];         // token-major e4m3 rows
  uint8_t vt[ATT_DV * ATT_VROW];         // dim-major e4m3 values
  uint16_t p[ATT_HPW * ATT_PROW];        // bf16 P[head][token]
  int slot[ATT_CH];
  float kscale[ATT_CH];
  float bias[ATT_CH];
  float red[4][ATT_HPW];
};

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

__global__ __launch_bounds__(ATT_THREADS) void sparse_mla_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv, const float* __restrict__ kvs,
    const int* __restrict__ idx, const int* __restrict__ cnt, const int* __restrict__ table,
    const int* __restrict__ rows, const float* __restrict__ bias, uint16_t* __restrict__ out,
    float* __restrict__ out_f32, float* __restrict__ lse_out, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    int B, int H, int keep, int max_pages, int page_size, int num_pages, float scale, int splits,
    int slots_per_split) {
  __shared__ AttShared sh;
  const int HG = H / ATT_HPW;
  const int groups = B * splits;
  // XCD-aware order: workgroup x runs on XCD x % 8; the HG head groups of one (sequence, split) read the same rows,
  // so they get ids that are equal mod 8 (the same XCD, the same L2).
  const int x = blockIdx.x;
  const int blk = x / (8 * HG), rem = x - blk * 8 * HG;
  const int hg = rem / 8;
  const int gi = blk * 8 + (rem - hg * 8);
  if (gi >= groups) return;
  const int b = gi / splits, sp = gi - b * splits;

  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int l16 = lane & 15, q4 = lane >> 4;
  const bool token_form = rows == nullptr;
  int n_eff = keep;
  if (token_form) {
    int c = cnt[b];
    c = c < 1 ? 1 : (c > keep ? keep : c);  // cnt 0: attend slot 0, fully masked (the reference's uniform row)
    n_eff = c;
  }
  const int k_begin = sp * slots_per_split;
  const int k_end = min(k_begin + slots_per_split, n_eff);

  // query operand: head 16hg + l16, dims 144 q4 + 8 st .. + 7 at step st
  const int head_b = ATT_HPW * hg + l16;
  bf16x8 qb[18];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(q + ((size_t)b * H + head_b) * ATT_DQK + 144 * q4);
#pragma unroll
    for (int st = 0; st < 18; ++st) qb[st] = as_bf16x8(qp[st]);
  }

  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // running max of head l16 (the same in every wave)
  float l_run = 0.0f;       // this lane's share of the running sum of head l16

  const int* trow = table ? table + (size_t)b * max_pages : nullptr;
  for (int k0 = k_begin; k0 < k_end; k0 += ATT_CH) {
    // slots, scales and biases of the chunk
    if (tid < ATT_CH) {
      const int k = k0 + tid;
      int slot = 0;
      float bs = NEG_INF;
      if (k < k_end) {
        if (token_form) {
          int pos = idx[(size_t)b * keep + k];
          pos = pos < 0 ? 0 : pos;
          int pi = pos / page_size;
          pi = pi < max_pages ? pi : max_pages - 1;
          slot = safe_page(trow[pi], num_pages) * page_size + (pos - (pos / page_size) * page_size);
          bs = (k < cnt[b]) ? 0.0f : NEG_INF;
        } else {
          slot = rows[(size_t)b * keep + k];
          slot = ((unsigned)slot < (unsigned)(num_pages * page_size)) ? slot : 0;
          bs = bias[(size_t)b * keep + k];
        }
      } else {
        // past the split: a copy of the chunk's first row with weight exactly 0 (bias -inf), also when every real
        // slot of the chunk is masked at NEG_INF (a fully masked row averages its real slots only)
        slot = -1;
        bs = -INFINITY;
      }
      sh.slot[tid] = slot;
      sh.bias[tid] = bs;
    }
    __syncthreads();
    if (tid < ATT_CH) {
      int slot = sh.slot[tid];
      if (slot < 0) slot = sh.slot[0];
      sh.slot[tid] = slot;
      sh.kscale[tid] = kvs[slot];
    }
    __syncthreads();
    // token-major staging: 64 rows x 36 pieces of 16 bytes
    for (int i = tid; i < ATT_CH * 36; i += ATT_THREADS) {
      const int r = i / 36, c = i - r * 36;
      const uint4 v = *reinterpret_cast<const uint4*>(kv + (size_t)sh.slot[r] * ATT_DQK + 16 * c);
      *reinterpret_cast<uint4*>(&sh.kt[r * ATT_KROW + 16 * c]) = v;
    }
    __syncthreads();
    // dim-major staging of the first 512 columns: 16 token quads x 128 dim quads, a 4x4 byte transpose each
    for (int i = tid; i < 16 * 128; i += ATT_THREADS) {
      const int g = i & 127, tq = i >> 7;
      uint32_t w0 = *reinterpret_cast<const uint32_t*>(&sh.kt[(4 * tq + 0) * ATT_KROW + 4 * g]);
      uint32_t w1 = *reinterpret_cast<const uint32_t*>(&sh.kt[(4 * tq + 1) * ATT_KROW + 4 * g]);
      uint32_t w2 = *reinterpret_cast<const uint32_t*>(&sh.kt[(4 * tq + 2) * ATT_KROW + 4 * g]);
      uint32_t w3 = *reinterpret_cast<const uint32_t*>(&sh.kt[(4 * tq + 3) * ATT_KROW + 4 * g]);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t t = byte_of(w0, d) | (byte_of(w1, d) << 8) | (byte_of(w2, d) << 16) | (byte_of(w3, d) << 24);
        *reinterpret_cast<uint32_t*>(&sh.vt[(4 * g + d) * ATT_VROW + 4 * tq]) = t;
      }
    }

    // scores of tokens 16 wave .. 16 wave + 15, heads l16
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    {
      const uint8_t* kr = &sh.kt[(16 * wave + l16) * ATT_KROW + 144 * q4];
#pragma unroll
      for (int st = 0; st < 18; ++st) {
        const uint2 kb = *reinterpret_cast<const uint2*>(kr + 8 * st);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kb.x, kb.y), qb[st], acc, 0, 0, 0);
      }
    }
    // acc[r] = S^T[token 16 wave + 4 q4 + r][head l16]
    float s[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tk = 16 * wave + 4 * q4 + r;
      s[r] = acc[r] * (sh.kscale[tk] * scale) + sh.bias[tk];
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
    if (lane < ATT_HPW) sh.red[wave][lane] = mx;
    __syncthreads();  // chunk maxima and both staged tiles visible
    float mc = fmaxf(fmaxf(sh.red[0][l16], sh.red[1][l16]), fmaxf(sh.red[2][l16], sh.red[3][l16]));
    const float m_new = fmaxf(m_run, mc);
    const float alpha = __expf(m_run - m_new);
    m_run = m_new;
    float psum = 0.0f;
    uint32_t pk[2];
#pragma unroll
    for (int r = 0; r < 4; r += 2) {
      const int tk = 16 * wave + 4 * q4 + r;
      const float p0 = __expf(s[r] - m_new), p1 = __expf(s[r + 1] - m_new);
      psum += p0 + p1;
      pk[r / 2] = (uint32_t)f32_to_bf16_bits(p0 * sh.kscale[tk]) |
                  ((uint32_t)f32_to_bf16_bits(p1 * sh.kscale[tk + 1]) << 16);
    }
    l_run = l_run * alpha + psum;
    *reinterpret_cast<uint2*>(&sh.p[l16 * ATT_PROW + 16 * wave + 4 * q4]) = make_uint2(pk[0], pk[1]);
    __syncthreads();  // P complete

    // rescale O (rows = heads 4 q4 + r) and accumulate P . V over the chunk's 64 tokens
    float al[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * q4 + r, WAVE);
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[n][r] *= al[r];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int tb = 32 * ks + 4 * q4;
      const uint2 pa = *reinterpret_cast<const uint2*>(&sh.p[l16 * ATT_PROW + tb]);
      const uint2 pb = *reinterpret_cast<const uint2*>(&sh.p[l16 * ATT_PROW + tb + 16]);
      const bf16x8 pop = as_bf16x8(make_uint4(pa.x, pa.y, pb.x, pb.y));
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int dim = 128 * wave + 16 * n + l16;
        const uint32_t va = *reinterpret_cast<const uint32_t*>(&sh.vt[dim * ATT_VROW + tb]);
        const uint32_t vb = *reinterpret_cast<const uint32_t*>(&sh.vt[dim * ATT_VROW + tb + 16]);
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, fp8x8_to_bf16x8(va, vb), o[n], 0, 0, 0);
      }
    }
    __syncthreads();  // the next chunk overwrites the tiles
  }

  // the row sums: lane shares -> per wave -> per workgroup
  float lw = l_run;
  lw += __shfl_xor(lw, 16, WAVE);
  lw += __shfl_xor(lw, 32, WAVE);
  if (lane < ATT_HPW) sh.red[wave][lane] = lw;
  __syncthreads();
  const float l_tot = sh.red[0][l16] + sh.red[1][l16] + sh.red[2][l16] + sh.red[3][l16];
  float lr[4], mr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lr[r] = __shfl(l_tot, 4 * q4 + r, WAVE);
    mr[r] = __shfl(m_run, 4 * q4 + r, WAVE);
  }
  const bool empty = k_begin >= k_end;
  if (splits == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = ATT_HPW * hg + 4 * q4 + r;
      const float inv = 1.0f / lr[r];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int dim = 128 * wave + 16 * n + l16;
        const float v = o[n][r] * inv;
        const size_t oi = ((size_t)b * H + head) * ATT_DV + dim;
        if (out) out[oi] = f32_to_bf16_bits(v);
        if (out_f32) out_f32[oi] = v;
      }
      if (lse_out && wave == 0 && l16 == 0) lse_out[(size_t)b * H + head] = mr[r] + __logf(lr[r]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = ATT_HPW * hg + 4 * q4 + r;
      const float inv = empty ? 0.0f : 1.0f / lr[r];
      const size_t base = (((size_t)b * splits + sp) * H + head) * ATT_DV;
#pragma unroll
      for (int n = 0; n < 8; ++n) ws_o[base + 128 * wave + 16 * n + l16] = o[n][r] * inv;
      // the split's running max and sum, not its lse: at a fully masked row lse = -1e30 + log(sum) rounds to -1e30
      // in fp32 and would lose the sums that weight the splits
      if (wave == 0 && l16 == 0) {
        const size_t mi = (((size_t)b * splits + sp) * H + head) * 2;
        ws_ml[mi] = empty ? -INFINITY : mr[r];
        ws_ml[mi + 1] = empty ? 0.0f : lr[r];
      }
    }
  }
}

// o = sum_s W_s o_s / sum_s W_s with W_s = l_s exp(m_s - M), M = max_s m_s, and lse = M + log sum_s W_s, per
// (sequence, head), from each split's normalised o_s, max m_s and sum l_s (the log-sum-exp combine of
// trnrt/models/mla.py:853-856 with lse_s = m_s + log l_s kept in two parts); 128 threads x 4 dims.
__global__ __launch_bounds__(128) void combine_splits_kernel(const float* __restrict__ ws_o,
                                                             const float* __restrict__ ws_ml, int H, int splits,
                                                             uint16_t* __restrict__ out, float* __restrict__ out_f32,
                                                             float* __restrict__ lse_out) {
  const int bh = blockIdx.x;
  const int b = bh / H, head = bh - b * H;
  float M = -INFINITY;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, ws_ml[(((size_t)b * splits + s) * H + head) * 2]);
  float W = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const int d = 4 * threadIdx.x;
  for (int s = 0; s < splits; ++s) {
    const size_t mi = (((size_t)b * splits + s) * H + head) * 2;
    const float ls = ws_ml[mi + 1];
    const float wt = ls > 0.0f ? ls * __expf(ws_ml[mi] - M) : 0.0f;
    W += wt;
    if (wt != 0.0f) {
      const float4 v = *reinterpret_cast<const float4*>(&ws_o[(((size_t)b * splits + s) * H + head) * ATT_DV + d]);
      acc.x += wt * v.x;
      acc.y += wt * v.y;
      acc.z += wt * v.z;
      acc.w += wt * v.w;
    }
  }
  const float inv = 1.0f / W;
  const size_t oi = ((size_t)b * H + head) * ATT_DV + d;
  if (out) {
    const uint32_t lo = f32_to_bf16_bits(acc.x * inv) | ((uint32_t)f32_to_bf16_bits(acc.y * inv) << 16);
    const uint32_t hi = f32_to_bf16_bits(acc.z * inv) | ((uint32_t)f32_to_bf16_bits(acc.w * inv) << 16);
    *reinterpret_cast<uint2*>(&out[oi]) = make_uint2(lo, hi);
  }
  if (out_f32) *reinterpret_cast<float4*>(&out_f32[oi]) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  if (lse_out && threadIdx.x == 0) lse_out[(size_t)b * H + head] = M + __logf(W);
}

// Token positions -> cache slots and biases (the kp = 1 form of trnrt/models/dsa_long.py:189-215).
__global__ void token_rows_kernel(const int* __restrict__ idx, const int* __restrict__ cnt,
                                  const int* __restrict__ table, int* __restrict__ rows, float* __restrict__ bias,
                                  int keep, int max_pages, int page_size, int num_pages) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= keep) return;
  const bool live = k < cnt[b];
  int pos = live ? idx[(size_t)b * keep + k] : 0;
  pos = pos < 0 ? 0 : pos;
  int pi = pos / page_size;
  pi = pi < max_pages ? pi : max_pages - 1;
  const int page = safe_page(table[(size_t)b * max_pages + pi], num_pages);
  rows[(size_t)b * keep + k] = page * page_size + pos % page_size;
  if (bias) bias[(size_t)b * keep + k] = live ? 0.0f : NEG_INF;
}

int attention_default_splits(int B, int H, int keep, int num_cu) {
  const int wgs = B * (H / ATT_HPW);
  const int max_splits = (keep + ATT_CH - 1) / ATT_CH;
  int s = (num_cu + wgs - 1) / (wgs > 0 ? wgs : 1);
  s = s < 1 ? 1 : s;
  return s > max_splits ? max_splits : s;
}

size_t attention_workspace_bytes(int B, int H, int splits) {
  if (splits <= 1) return 0;
  return (size_t)B * splits * H * ATT_DV * 4 + (size_t)B * splits * H * 8 + 256;
}

hipError_t launch_sparse_mla(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* idx, const int* cnt,
                             const int* table, const int* rows, const float* bias, uint16_t* out, float* out_f32,
                             float* lse, void* ws, int B, int H, int keep, int max_pages, int page_size,
                             int num_pages, float scale, int splits, hipStream_t s) {
  const int HG = H / ATT_HPW;
  // slots per split: a whole number of chunks
  int sps = (keep + splits - 1) / splits;
  sps = (sps + ATT_CH - 1) / ATT_CH * ATT_CH;
  const int eff_splits = (keep + sps - 1) / sps;
  const int groups = B * eff_splits;
  const int grid = (groups + 7) / 8 * 8 * HG;
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
  if (eff_splits > 1) {
    ws_o = static_cast<float*>(ws);
    ws_ml = ws_o + (size_t)B * eff_splits * H * ATT_DV;  // [B, splits, H, 2]: max, sum
  }
  hipLaunchKernelGGL(sparse_mla_kernel, dim3(grid), dim3(ATT_THREADS), 0, s, q, kv, kvs, idx, cnt, table, rows, bias,
                     out, out_f32, lse, ws_o, ws_ml, B, H, keep, max_pages, page_size, num_pages, scale, eff_splits,
                     sps);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || eff_splits == 1) return e;
  hipLaunchKernelGGL(combine_splits_kernel, dim3(B * H), dim3(128), 0, s, ws_o, ws_ml, H, eff_splits, out, out_f32,
                     lse);
  return hipGetLastError();
}

hipError_t launch_token_rows(const int* idx, const int* cnt, const int* table, int* rows, float* bias, int B,
                             int keep, int max_pages, int page_size, int num_pages, hipStream_t s) {
  hipLaunchKernelGGL(token_rows_kernel, dim3((keep + 255) / 256, B), dim3(256), 0, s, idx, cnt, table, rows, bias,
                     keep, max_pages, page_size, num_pages);
  return hipGetLastError();
}

}  // namespace dsa
