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
constexpr int ATT_SUPER = 256;    // slots whose ids / scales / biases are set up at once (one per thread)
constexpr int ATT_PIECES = ATT_DQK / 16;  // 16-byte pieces of a row
constexpr int ATT_RPT = ATT_CH * ATT_PIECES / ATT_THREADS;  // pieces per thread per chunk (9)
// Token-major row stride: 146 dwords, so the staging writes, the score operand reads and the transposing value
// reads of rows 0..31 spread over the banks (at most 2-way).
constexpr int ATT_KROW = ATT_DQK + 8;   // bytes
constexpr int ATT_PROW = ATT_CH + 8;    // P row stride (bf16 elements; 16-byte aligned rows)

typedef int att_v2i __attribute__((ext_vector_type(2)));

struct AttShared {
  uint8_t kt[ATT_CH * ATT_KROW];   // token-major e4m3 rows of the chunk
  uint16_t p[ATT_HPW * ATT_PROW];  // bf16 P[head][token]
  int slot[ATT_SUPER];
  float kscale[ATT_SUPER];
  float bias[ATT_SUPER];
  float red[4][ATT_HPW];
};

// The value operand of v_mfma_f32_16x16x32_bf16 straight from the token-major tile: ds_read_b64_tr_b8 gives lane
// (a = i / 8, c = i % 8) of each 16-lane block byte c of the 8-byte rows addressed by the block's lanes 2j + a,
// j = 0..7. Lane p of block q addresses token 32 ks + 8 q + p / 2 at dims 16 n + 8 (p & 1), so lane l receives dim
// 16 n + l % 16 of tokens 32 ks + 8 (l / 16) + j: the B operand with k-slot 8 q + j = that token.
__device__ __forceinline__ bf16x8 value_operand(const uint8_t* kt, int ks, int n, int lane) {
  const int q = lane >> 4, p = lane & 15;
  const uint8_t* a = kt + (32 * ks + 8 * q + (p >> 1)) * ATT_KROW + 16 * n + 8 * (p & 1);
  const att_v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) att_v2i*)(a));
  return fp8x8_to_bf16x8((uint32_t)r.x, (uint32_t)r.y);
}

__global__ __launch_bounds__(ATT_THREADS, 2) void sparse_mla_kernel(
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
  int cnt_b = keep;
  if (token_form) {
    cnt_b = cnt[b];
    int c = cnt_b < 1 ? 1 : (cnt_b > keep ? keep : cnt_b);  // cnt 0: attend slot 0, fully masked
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
  for (int sc0 = k_begin; sc0 < k_end; sc0 += ATT_SUPER) {
    const int nslots = min(ATT_SUPER, k_end - sc0);
    const int nch = (nslots + ATT_CH - 1) / ATT_CH;
    // slots, scales and biases of the super-chunk: one per thread
    {
      const int k = sc0 + tid;
      int slot = -1;
      float bs = -INFINITY;  // past the split: weight exactly 0 (a copy of the super-chunk's first row)
      if (tid < nslots) {
        if (token_form) {
          int pos = idx[(size_t)b * keep + k];
          pos = pos < 0 ? 0 : pos;
          int pi = pos / page_size;
          pi = pi < max_pages ? pi : max_pages - 1;
          slot = safe_page(trow[pi], num_pages) * page_size + (pos - (pos / page_size) * page_size);
          bs = (k < cnt_b) ? 0.0f : NEG_INF;
        } else {
          slot = rows[(size_t)b * keep + k];
          slot = ((unsigned)slot < (unsigned)(num_pages * page_size)) ? slot : 0;
          bs = bias[(size_t)b * keep + k];
        }
      }
      sh.slot[tid] = slot;
      sh.bias[tid] = bs;
      __syncthreads();
      if (slot < 0) slot = sh.slot[0];  // slot 0 of a super-chunk is always real
      __syncthreads();
      sh.slot[tid] = slot;
      sh.kscale[tid] = kvs[slot];
    }
    __syncthreads();
    // the chunk's rows in registers (thread tid holds 16-byte pieces tid + 256 j), one chunk ahead of the tile
    uint4 rv[ATT_RPT];
    auto load_rows = [&](int c) {
#pragma unroll
      for (int jj = 0; jj < ATT_RPT; ++jj) {
        const int i = tid + ATT_THREADS * jj;
        const int r = i / ATT_PIECES, pc = i - r * ATT_PIECES;
        rv[jj] = *reinterpret_cast<const uint4*>(kv + (size_t)sh.slot[c * ATT_CH + r] * ATT_DQK + 16 * pc);
      }
    };
    load_rows(0);

    for (int c = 0; c < nch; ++c) {
      const int cb = c * ATT_CH;  // the chunk's first slot inside the super-chunk
#pragma unroll
      for (int jj = 0; jj < ATT_RPT; ++jj) {
        const int i = tid + ATT_THREADS * jj;
        const int r = i / ATT_PIECES, pc = i - r * ATT_PIECES;
        uint8_t* dst = &sh.kt[r * ATT_KROW + 16 * pc];
        *reinterpret_cast<uint2*>(dst) = make_uint2(rv[jj].x, rv[jj].y);
        *reinterpret_cast<uint2*>(dst + 8) = make_uint2(rv[jj].z, rv[jj].w);
      }
      __syncthreads();  // the tile is complete
      if (c + 1 < nch) load_rows(c + 1);  // the next chunk's loads fly while this one computes

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
      float s4[4];
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = cb + 16 * wave + 4 * q4 + r;
        s4[r] = acc[r] * (sh.kscale[tk] * scale) + sh.bias[tk];
        mx = fmaxf(mx, s4[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
      mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
      if (lane < ATT_HPW) sh.red[wave][lane] = mx;
      __syncthreads();  // the chunk maxima
      const float mc = fmaxf(fmaxf(sh.red[0][l16], sh.red[1][l16]), fmaxf(sh.red[2][l16], sh.red[3][l16]));
      const float m_new = fmaxf(m_run, mc);
      const float alpha = __expf(m_run - m_new);
      m_run = m_new;
      float psum = 0.0f;
      uint32_t pk[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int tk = cb + 16 * wave + 4 * q4 + r;
        const float p0 = __expf(s4[r] - m_new), p1 = __expf(s4[r + 1] - m_new);
        psum += p0 + p1;
        pk[r / 2] = (uint32_t)f32_to_bf16_bits(p0 * sh.kscale[tk]) |
                    ((uint32_t)f32_to_bf16_bits(p1 * sh.kscale[tk + 1]) << 16);
      }
      l_run = l_run * alpha + psum;
      *reinterpret_cast<uint2*>(&sh.p[l16 * ATT_PROW + 16 * wave + 4 * q4]) = make_uint2(pk[0], pk[1]);
      __syncthreads();  // P complete

      // rescale O (rows = heads 4 q4 + r) and accumulate P . V over the chunk's 64 tokens (dims 128 wave ..)
      float al[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * q4 + r, WAVE);
#pragma unroll
      for (int n = 0; n < 8; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[n][r] *= al[r];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // P operand: head l16, tokens 32 ks + 8 q4 .. + 7 (the value operand's k-slot order)
        const bf16x8 pop = as_bf16x8(*reinterpret_cast<const uint4*>(&sh.p[l16 * ATT_PROW + 32 * ks + 8 * q4]));
#pragma unroll
        for (int n = 0; n < 8; ++n)
          o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, value_operand(sh.kt, ks, 8 * wave + n, lane), o[n], 0,
                                                         0, 0);
      }
      __syncthreads();  // the next chunk overwrites the tiles
    }
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
// trnrt/models/mla.py:853-856 with lse_s = m_s + log l_s kept in two parts); 128 threads x 4 dims. Every load is
// issued before any is used (one memory round trip); an empty split's o_s is 0 and its weight 0.
template <int S>
__global__ __launch_bounds__(128) void combine_splits_kernel(const float* __restrict__ ws_o,
                                                             const float* __restrict__ ws_ml, int H, int splits,
                                                             uint16_t* __restrict__ out, float* __restrict__ out_f32,
                                                             float* __restrict__ lse_out) {
  const int bh = blockIdx.x;
  const int b = bh / H, head = bh - b * H;
  const int d = 4 * threadIdx.x;
  float2 ml[S];
  float4 v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s < splits) {
      const size_t i = ((size_t)b * splits + s) * H + head;
      ml[s] = *reinterpret_cast<const float2*>(&ws_ml[2 * i]);
      v[s] = *reinterpret_cast<const float4*>(&ws_o[i * ATT_DV + d]);
    } else {
      ml[s] = make_float2(-INFINITY, 0.0f);
      v[s] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[s].x);
  float W = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float wt = ml[s].y > 0.0f ? ml[s].y * __expf(ml[s].x - M) : 0.0f;
    W += wt;
    acc.x += wt * v[s].x;
    acc.y += wt * v[s].y;
    acc.z += wt * v[s].z;
    acc.w += wt * v[s].w;
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
  int max_splits = (keep + ATT_CH - 1) / ATT_CH;
  max_splits = max_splits > 32 ? 32 : max_splits;
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
  launch("sparse_mla_kernel", sparse_mla_kernel, dim3(grid), dim3(ATT_THREADS), s, q, kv, kvs, idx, cnt, table, rows, bias,
                     out, out_f32, lse, ws_o, ws_ml, B, H, keep, max_pages, page_size, num_pages, scale, eff_splits,
                     sps);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || eff_splits == 1) return e;
  if (eff_splits <= 8)
    launch("combine_splits_kernel", combine_splits_kernel<8>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H, eff_splits, out,
                       out_f32, lse);
  else if (eff_splits <= 16)
    launch("combine_splits_kernel", combine_splits_kernel<16>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H, eff_splits, out,
                       out_f32, lse);
  else
    launch("combine_splits_kernel", combine_splits_kernel<32>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H, eff_splits, out,
                       out_f32, lse);
  return hipGetLastError();
}

hipError_t launch_token_rows(const int* idx, const int* cnt, const int* table, int* rows, float* bias, int B,
                             int keep, int max_pages, int page_size, int num_pages, hipStream_t s) {
  launch("token_rows_kernel", token_rows_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, table, rows, bias,
                     keep, max_pages, page_size, num_pages);
  return hipGetLastError();
}

}  // namespace dsa
