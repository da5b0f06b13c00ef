// Sparse MLA decode attention for gfx950 over the selected tokens of a paged FP8 latent cache (the arithmetic of
// trnrt/kernels/dsa_decode.py:26-37 and trnrt/kernels/dsa_slots.py:48-65, absorbed MLA, with a 576-wide key of
// 512 latent + 64 rope columns, or GLM's 512-wide NoPE latent, and the first 512 columns as the value; per-token FP8
// scales):
//
//   s[h, k] = scale * q[h, :] . K[k] + bias[k],  K[k] = kv_fp8[slot_k] * kv_scale[slot_k]
//   o[h, :] = sum_k softmax_k(s)[h, k] * K[k][:512],  lse[h] = max_k s + log sum_k exp(s - max)
//
// Work unit: one workgroup = one sequence, 16 query heads, one split of the selected slots (split-K), 8 waves.
// The split's slot ids and the queries come in one round of loads; then the rows of up to 256 slots (4 chunks of 64)
// are gathered straight into LDS by direct-to-LDS loads (global_load_lds_dwordx4: consecutive lanes read
// consecutive 16-byte pieces of a row, no register staging), all issued at once, so the workgroup waits for memory
// twice: slot ids, then rows. A chunk is token-major e4m3 with a 592-byte row stride (36 pieces and one padding
// piece, filled with a copy of piece 35), which spreads the operand reads over the LDS banks. Both products run on
// v_mfma_f32_16x16x32_bf16 with e4m3 -> bf16 conversions in registers (exact):
//   - scores: S^T[token, head] = K . Q^T; 16 tokens per wave, all 16 heads, the 576 dims in 18 steps of 32 (at each
//     step the four lane groups read consecutive 8-byte pieces of a row, so lanes 0-31 and 32-63 each cover every
//     LDS bank once; q staged once through LDS);
//   - online softmax in fp32 with the chunk maximum shared through LDS;
//   - value: O[head, dim] += P . V with P = exp(s - m) * kv_scale rounded to bf16 (the dequantisation of the value
//     folded into the weight), its operand read transposed from the token-major rows by ds_read_b64_tr_b8.
// The two halves of the workgroup (waves 0-3, 4-7) take alternate chunks, each with its own running max, sum and
// output, merged at the end; within a half, wave w takes tokens 16w .. 16w + 15 for the scores and dims
// 128w .. 128w + 127 for the value product.
// With one split the workgroup writes bf16 o and lse; with several it writes fp32 partial o (normalised) with its
// running max and sum, and a combine kernel merges them by log-sum-exp (trnrt/models/mla.py:853-856, 1152-1160).
#include "dsa_common.h"

namespace dsa {

constexpr int ATT_DV = 512;      // the value: the first 512 columns of a row (the latent)
constexpr int ATT_HPW = 16;       // heads per workgroup
constexpr int ATT_CH = 64;        // slots per chunk
constexpr int ATT_THREADS = 512;  // 8 waves: two halves of 4
constexpr int ATT_NCH = 4;        // chunks staged in LDS at once
constexpr int ATT_SUPER = ATT_NCH * ATT_CH;  // slots staged at once
// Rows of DQK = 576 (512 latent + 64 rope, 36 16-byte pieces) or 512 (a NoPE latent, 32 pieces) columns; in LDS
// both take 37 pieces (592 bytes: the data and one or five padding pieces), the stride that spreads the operand
// reads over the banks.
constexpr int ATT_KPIECES = 37;
constexpr int ATT_KROW = 16 * ATT_KPIECES;   // 592 bytes
constexpr int ATT_CHUNK_BYTES = ATT_CH * ATT_KROW;  // 37,888: 37 direct-to-LDS instructions of 1 KiB
constexpr int ATT_LOADS = ATT_NCH * ATT_KPIECES;    // 148 instructions per staged super-chunk
constexpr int ATT_PROW = ATT_CH + 8;         // P row stride (bf16 elements; 16-byte aligned rows)
constexpr int ATT_TAIL_BYTES = 3584;         // a pooled tail staged apart: 7 rows of 512 bytes or 6 of 576

typedef int att_v2i __attribute__((ext_vector_type(2)));

struct AttShared {
  uint8_t kt[ATT_NCH][ATT_CHUNK_BYTES];  // token-major e4m3 rows of the staged chunks (q before them)
  uint16_t p[2][ATT_HPW * ATT_PROW];     // per half: bf16 P[head][token]
  int slot[ATT_SUPER];
  float kscale[ATT_SUPER];
  float bias[ATT_SUPER];
  float red[2][4][ATT_HPW];
  float ml[2][ATT_HPW];  // the second half's final max and sum per head, for the merge
  int tslot[8];          // the pooled tail's cache slots (kpool <= 8: at most 7 tail tokens) and scales
  float tks[8];
  uint8_t trows[ATT_TAIL_BYTES];  // the pooled tail's rows, loaded with the first super-chunk's
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

// Slot forms: token (idx + cnt + table: positions through the page table, bias 0 below cnt), rows + bias (cache
// slots with an additive bias), rows + cnt (cache slots, bias 0 below cnt). The token form's pooled variant (pf.kp_shift
// > 0, kpool = 1 << kp_shift): idx [B, pf.idx_stride] selected pools, cnt their count; the row attends the kpool
// tokens of each selected pool and then the tail: tokens kpool npool .. pos of its incomplete pool npool (none when
// pos + 1 is a multiple of kpool), token slot k = pool slot k >> kp_shift, token k & (kpool - 1) of that pool -- the
// slots of trnrt/models/dsa_long.py:189-215 in the same order, with the masked ones left out.
template <int DQK>
__global__ __launch_bounds__(ATT_THREADS, 1) void sparse_mla_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv, const float* __restrict__ kvs,
    const int* __restrict__ idx, const int* __restrict__ cnt, const int* __restrict__ table,
    const int* __restrict__ rows, const float* __restrict__ bias, uint16_t* __restrict__ out,
    float* __restrict__ out_f32, float* __restrict__ lse_out, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    int B, int H, int keep, int max_pages, int page_size, int num_pages, float scale, int splits,
    int slots_per_split, PoolForm pf) {
  constexpr int ATT_PIECES = DQK / 16;  // 16-byte data pieces per row
  constexpr int ATT_QROW = DQK + 8;     // staged query row stride (bf16 elements)
  constexpr int STEPS = DQK / 32;       // score steps of 32 dims
  static_assert(ATT_PIECES < ATT_KPIECES && STEPS % 2 == 0, "row width");
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
  if (pf.n_live && b >= *pf.n_live) return;  // a row past the run-time live count: left unwritten

  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int half = wave >> 2, wh = wave & 3;  // the half (alternate chunks) and the wave within it
  const int l16 = lane & 15, q4 = lane >> 4;
  const bool token_form = rows == nullptr;
  int n_eff = keep;
  int cnt_b = keep;
  int pools_b = 0, tail_pool = 0;  // pooled form: selected pools, the tail pool
  int tail_apart = 0;              // pooled form with the tail apart: the row's tail tokens
  if (cnt) {
    cnt_b = cnt[b];
    if (pf.kp_shift) {
      // token slots: kpool per selected pool, then the tail's tokens
      pools_b = min(max(cnt_b, 0), pf.idx_stride);
      tail_pool = max(pf.npool[b], 0);
      const int tail = min(max(pf.positions[b] + 1 - (tail_pool << pf.kp_shift), 0), (1 << pf.kp_shift) - 1);
      cnt_b = pools_b << pf.kp_shift;
      if (pf.tail_apart)
        tail_apart = tail;
      else
        cnt_b += tail;
    }
    // cnt 0: attend slot 0 (or the first pf.empty_n slots), fully masked
    if (!bias) n_eff = cnt_b < 1 ? min(max(pf.empty_n, 1), keep) : (cnt_b > keep ? keep : cnt_b);
  }
  const int k_begin = sp * slots_per_split;
  const int k_end = min(k_begin + slots_per_split, n_eff);
  // the workgroup that holds the row's last slot (n_eff >= 1 here, so it has slots of its own) adds the tail as one
  // more chunk: rows 0 .. tail_n - 1 of a zeroed tile, loaded into registers with its first super-chunk's rows
  const int tail_n = (tail_apart > 0 && (n_eff - 1) / slots_per_split == sp) ? tail_apart : 0;
  const size_t nslots_cache = (size_t)num_pages * page_size;

  // the queries of the 16 heads (16 or 18 KiB), staged through LDS below
  const uint4* qsrc = reinterpret_cast<const uint4*>(q + ((size_t)b * H + ATT_HPW * hg) * DQK);
  constexpr int QPIECES = ATT_HPW * DQK / 8;  // 16-byte pieces: 1024 or 1152
  uint4 qv[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) qv[i] = qsrc[min(tid + ATT_THREADS * i, QPIECES - 1)];

  bf16x8 qb[STEPS];
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // running max of head l16 over this half's chunks (the same in its 4 waves)
  float l_run = 0.0f;       // this lane's share of the half's running sum of head l16

  const int* trow = table ? table + (size_t)b * max_pages : nullptr;
  // one pair of staged chunks: half h takes chunk c0 + h of the nch staged (tile c, slots 64 c .. of the super-chunk)
  auto chunk_pair = [&](int c0, int nch) __attribute__((always_inline)) {
    const int c = c0 + half;  // this half's chunk of the pair
    const bool live = c < nch;
    const int cb = c * ATT_CH;
    const uint8_t* kt = sh.kt[live ? c : 0];
    float s4[4];
    float alpha = 1.0f;
    if (live) {
      // scores of tokens 16 wh .. 16 wh + 15, heads l16 (two accumulators: independent MFMA chains); lane group q4
      // reads 16 bytes of its row per pair of steps (dims 64 j + 16 q4 ..: one ds_read_b128 for two MFMAs, 8 rows
      // at one column covering the 32 banks once at the 592-byte stride)
      f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
      const uint8_t* kr = kt + (16 * wh + l16) * ATT_KROW + 16 * q4;
#pragma unroll
      for (int st = 0; st < STEPS; st += 2) {
        const u32x4 kk = *reinterpret_cast<const u32x4*>(kr + 32 * st);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[0], kk[1]), qb[st], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[2], kk[3]), qb[st + 1], acc1, 0, 0, 0);
      }
      // acc[r] = S^T[token 16 wh + 4 q4 + r][head l16]
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = cb + 16 * wh + 4 * q4 + r;
        s4[r] = (acc0[r] + acc1[r]) * (sh.kscale[tk] * scale) + sh.bias[tk];
        mx = fmaxf(mx, s4[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
      mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
      if (lane < ATT_HPW) sh.red[half][wh][lane] = mx;
    }
    __syncthreads();  // the chunk maxima
    if (live) {
      const float mc = fmaxf(fmaxf(sh.red[half][0][l16], sh.red[half][1][l16]),
                             fmaxf(sh.red[half][2][l16], sh.red[half][3][l16]));
      const float m_new = fmaxf(m_run, mc);
      alpha = __expf(m_run - m_new);
      m_run = m_new;
      float psum = 0.0f;
      uint32_t pk[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int tk = cb + 16 * wh + 4 * q4 + r;
        const float p0 = __expf(s4[r] - m_new), p1 = __expf(s4[r + 1] - m_new);
        psum += p0 + p1;
        pk[r / 2] = (uint32_t)f32_to_bf16_bits(p0 * sh.kscale[tk]) |
                    ((uint32_t)f32_to_bf16_bits(p1 * sh.kscale[tk + 1]) << 16);
      }
      l_run = l_run * alpha + psum;
      *reinterpret_cast<uint2*>(&sh.p[half][l16 * ATT_PROW + 16 * wh + 4 * q4]) = make_uint2(pk[0], pk[1]);
    }
    __syncthreads();  // P complete (and every wave has read the maxima)
    if (live) {
      // rescale O (rows = heads 4 q4 + r) and accumulate P . V over the chunk's 64 tokens (dims 128 wh ..)
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
        const bf16x8 pop =
            as_bf16x8(*reinterpret_cast<const uint4*>(&sh.p[half][l16 * ATT_PROW + 32 * ks + 8 * q4]));
#pragma unroll
        for (int n = 0; n < 8; ++n)
          o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, value_operand(kt, ks, 8 * wh + n, lane), o[n], 0, 0,
                                                         0);
      }
    }
    // the next pair's maxima and P are written after its first barrier, which every wave reaches only after
    // this pair's P . V
  };
  for (int sc0 = k_begin; sc0 < k_end; sc0 += ATT_SUPER) {
    const int nslots = min(ATT_SUPER, k_end - sc0);
    const int nch = (nslots + ATT_CH - 1) / ATT_CH;
    const bool tail_thread = sc0 == k_begin && tid >= ATT_SUPER && tid - ATT_SUPER < tail_n;
    // slot ids and biases, one per thread of the first 256 (past the split: slot 0's row with weight exactly 0)
    if (tail_thread) {
      // the tail tokens' cache slots, with the first super-chunk's
      const int pos = (tail_pool << pf.kp_shift) + (tid - ATT_SUPER);
      int pi = pos / page_size;
      pi = pi < max_pages ? pi : max_pages - 1;
      sh.tslot[tid - ATT_SUPER] = safe_page(trow[pi], num_pages) * page_size + (pos - (pos / page_size) * page_size);
    }
    if (tid < ATT_SUPER) {
      const int k = min(sc0 + tid, keep - 1);
      int slot;
      float bs;
      if (token_form) {
        int pos;
        if (pf.kp_shift) {
          const int j = k >> pf.kp_shift;
          const int pool = j < pools_b ? idx[(size_t)b * pf.idx_stride + j] : tail_pool;
          pos = (pool << pf.kp_shift) + (k & ((1 << pf.kp_shift) - 1));
        } else {
          pos = idx[(size_t)b * keep + k];
        }
        pos = pos < 0 ? 0 : pos;
        int pi = pos / page_size;
        pi = pi < max_pages ? pi : max_pages - 1;
        slot = safe_page(trow[pi], num_pages) * page_size + (pos - (pos / page_size) * page_size);
        bs = (k < cnt_b) ? 0.0f : NEG_INF;
      } else {
        slot = rows[(size_t)b * keep + k];
        slot = ((size_t)(unsigned)slot < nslots_cache) ? slot : 0;
        bs = bias ? bias[(size_t)b * keep + k] : ((k < cnt_b) ? 0.0f : NEG_INF);
      }
      sh.slot[tid] = slot;
      sh.bias[tid] = tid < nslots ? bs : -INFINITY;
    }
    __syncthreads();
    if (sc0 == k_begin) {
      // query operand: head 16hg + l16, dims 32 st + 8 q4 .. + 7 at step st, through the rows' LDS (q rows padded
      // by 8 elements so the operand reads spread over the banks)
      uint16_t* qs = reinterpret_cast<uint16_t*>(sh.kt[ATT_NCH - 1]);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int pc = tid + ATT_THREADS * i;  // 16-byte piece: head pc / (DQK / 8), elements 8 (pc % (DQK / 8)) ..
        if (pc < QPIECES)
          *reinterpret_cast<uint4*>(qs + (pc / (DQK / 8)) * ATT_QROW + 8 * (pc % (DQK / 8))) = qv[i];
      }
      __syncthreads();
      // in the key operand's dim order: steps 2 j, 2 j + 1 give lane group q4 dims 64 j + 16 q4 + 8 (st % 2) .. + 7
      const uint16_t* qh = qs + l16 * ATT_QROW + 16 * q4;
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
        qb[st] = as_bf16x8(*reinterpret_cast<const uint4*>(qh + 64 * (st >> 1) + 8 * (st & 1)));
      __syncthreads();  // every wave holds its operand before the rows overwrite it
    }
    // every staged row straight into LDS: instruction kk (chunk kk / 37, 1-KiB block j = kk % 37 of its tile) has
    // lane l load 16-byte unit u = 64 j + l of the tile: row u / 37, piece u % 37 (a padding piece re-reads the
    // last data piece);
    // the 148 instructions are spread over the 8 waves
    {
      int src_slot[(ATT_LOADS + 7) / 8];
#pragma unroll
      for (int i = 0; i < (ATT_LOADS + 7) / 8; ++i) {
        const int kk = min(wave + 8 * i, ATT_LOADS - 1);
        const int c = kk / ATT_KPIECES, j = kk - c * ATT_KPIECES;
        const int rr = c * ATT_CH + (WAVE * j + lane) / ATT_KPIECES;
        src_slot[i] = sh.slot[rr < nslots ? rr : 0];
      }
#pragma unroll
      for (int i = 0; i < (ATT_LOADS + 7) / 8; ++i) {
        const int kk = wave + 8 * i;
        const int c = kk / ATT_KPIECES, j = kk - c * ATT_KPIECES;
        if (kk < ATT_LOADS && c < nch) {
          const int u = WAVE * j + lane;
          const int pc = u - (u / ATT_KPIECES) * ATT_KPIECES;
          const uint8_t* src = kv + (size_t)src_slot[i] * DQK + 16 * (pc < ATT_PIECES ? pc : ATT_PIECES - 1);
          __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&sh.kt[c][1024 * j], 16, 0,
                                           0);
        }
      }
    }
    // the tail rows straight into their own LDS (rows of DQK bytes), beside the first super-chunk's rows: lane l of
    // wave w < 4 loads piece 64 w + l of the tail
    if (sc0 == k_begin && wave < 4) {
      const int u = WAVE * wave + lane;
      if (u < tail_n * ATT_PIECES)
        __builtin_amdgcn_global_load_lds(kv + (size_t)sh.tslot[u / ATT_PIECES] * DQK + 16 * (u % ATT_PIECES),
                                         (__attribute__((address_space(3))) void*)&sh.trows[1024 * wave], 16, 0, 0);
    }
    // (kvs null: the reference's unscaled cache, scale 1)
    const float ksc = tid < ATT_SUPER ? (kvs ? kvs[sh.slot[tid < nslots ? tid : 0]] : 1.0f)
                                      : (tail_thread ? (kvs ? kvs[sh.tslot[tid - ATT_SUPER]] : 1.0f) : 0.0f);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's rows are in LDS
    if (tid < ATT_SUPER)
      sh.kscale[tid] = ksc;
    else if (tail_thread)
      sh.tks[tid - ATT_SUPER] = ksc;
    __syncthreads();  // every wave's rows are in LDS
    for (int c0 = 0; c0 < nch; c0 += 2) chunk_pair(c0, nch);
    __syncthreads();  // the next super-chunk overwrites the staged rows and slots
  }
  if (tail_n > 0) {
    // the tail chunk: its rows copied into tile 0, every other row of the tile zero (finite operands where the
    // weight is 0), scales and biases for 64 slots
    for (int i = tid; i < ATT_CH * ATT_KPIECES; i += ATT_THREADS)
      if (i / ATT_KPIECES >= tail_n) *reinterpret_cast<u32x4*>(&sh.kt[0][16 * i]) = u32x4{0u, 0u, 0u, 0u};
    if (tid < tail_n * ATT_PIECES)
      *reinterpret_cast<u32x4*>(&sh.kt[0][(tid / ATT_PIECES) * ATT_KROW + 16 * (tid % ATT_PIECES)]) =
          *reinterpret_cast<const u32x4*>(&sh.trows[16 * tid]);
    if (tid < ATT_CH) {
      sh.kscale[tid] = tid < tail_n ? sh.tks[tid] : 0.0f;
      sh.bias[tid] = tid < tail_n ? 0.0f : -INFINITY;
    }
    __syncthreads();
    chunk_pair(0, 1);
  }

  // each half's row sums: lane shares -> per wave -> per half
  float lw = l_run;
  lw += __shfl_xor(lw, 16, WAVE);
  lw += __shfl_xor(lw, 32, WAVE);
  if (lane < ATT_HPW) sh.red[half][wh][lane] = lw;
  __syncthreads();
  const float l_half = sh.red[half][0][l16] + sh.red[half][1][l16] + sh.red[half][2][l16] + sh.red[half][3][l16];
  // merge the halves: the second half hands its max, sum and output to the first through LDS (the staged rows are
  // no longer needed)
  float* xo = reinterpret_cast<float*>(sh.kt[0]);  // [4 waves][32 values][64 lanes]
  if (half == 1) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) xo[(wh * 32 + 4 * n + r) * WAVE + lane] = o[n][r];
    if (wh == 0 && lane < ATT_HPW) {
      sh.ml[0][lane] = m_run;
      sh.ml[1][lane] = l_half;
    }
  }
  __syncthreads();
  const bool writer = half == 0;  // the first half writes the merged result
  const float m1 = sh.ml[0][l16], l1 = sh.ml[1][l16];
  const float m_tot = fmaxf(m_run, m1);
  const float a0 = m_run == -INFINITY ? 0.0f : __expf(m_run - m_tot);
  const float a1 = m1 == -INFINITY ? 0.0f : __expf(m1 - m_tot);
  const float l_tot = a0 * l_half + a1 * l1;
  float lr[4], mr[4], a0r[4], a1r[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lr[r] = __shfl(l_tot, 4 * q4 + r, WAVE);
    mr[r] = __shfl(m_tot, 4 * q4 + r, WAVE);
    a0r[r] = __shfl(a0, 4 * q4 + r, WAVE);
    a1r[r] = __shfl(a1, 4 * q4 + r, WAVE);
  }
#pragma unroll
  for (int n = 0; n < 8; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[n][r] = a0r[r] * o[n][r] + a1r[r] * xo[(wh * 32 + 4 * n + r) * WAVE + lane];
  const bool empty = k_begin >= k_end;
  if (splits == 1) {
    if (writer) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int head = ATT_HPW * hg + 4 * q4 + r;
        const float inv = 1.0f / lr[r];
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const int dim = 128 * wh + 16 * n + l16;
          const float v = o[n][r] * inv;
          const size_t oi = ((size_t)b * H + head) * ATT_DV + dim;
          if (out) out[oi] = f32_to_bf16_bits(v);
          if (out_f32) out_f32[oi] = v;
        }
        if (lse_out && wh == 0 && l16 == 0) lse_out[(size_t)b * H + head] = mr[r] + __logf(lr[r]);
      }
    }
    return;
  }
  if (writer) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = ATT_HPW * hg + 4 * q4 + r;
      const float inv = empty ? 0.0f : 1.0f / lr[r];
      const size_t base = (((size_t)b * splits + sp) * H + head) * ATT_DV;
#pragma unroll
      for (int n = 0; n < 8; ++n) ws_o[base + 128 * wh + 16 * n + l16] = o[n][r] * inv;
      // the split's running max and sum, not its lse: at a fully masked row lse = -1e30 + log(sum) rounds to -1e30
      // in fp32 and would lose the sums that weight the splits
      if (wh == 0 && l16 == 0) {
        const size_t mi = (((size_t)b * splits + sp) * H + head) * 2;
        ws_ml[mi] = empty ? -INFINITY : mr[r];
        ws_ml[mi + 1] = empty ? 0.0f : lr[r];
      }
    }
  }
}

// The many-row form (a prefill chunk's query rows, or any launch with one split and at least a workgroup per CU):
// one workgroup = one query row x 64 heads over all its slots, so each gathered row serves 64 heads instead of 16,
// and the gather is pipelined: chunk c + 2's rows are loaded into registers while chunk c is computed (two register
// sets of LPT 16-byte pieces per thread, stored into two LDS tiles), so the workgroup waits for memory once at the
// start (slot ids, scales, queries) instead of once per 256 slots. The 8 waves split the work as
//   - scores: wave (hg = w % 4, th = w / 4) takes heads 16 hg .. + 15 and half th of the dims (9 or 8 steps of 32)
//     over all 64 tokens of the chunk (S^T = K . Q^T on v_mfma_f32_16x16x32_bf16, four token blocks as independent
//     chains), the query operand of its heads and dims in registers for the whole row (36 or 32 registers: the full
//     width would not fit beside the output and the gather registers); the two halves' partial scores are
//     exchanged through LDS, so both waves of a head group hold the chunk's full scores;
//   - softmax: each wave takes the chunk maximum of its heads over all 64 tokens, P = exp(s - m) * kv_scale in bf16
//     for its 32 tokens (32 th ..) into LDS [64 heads][64 tokens], the rescale factors into LDS;
//   - value: wave w takes dims 64 w .. 64 w + 63 of all 64 heads (O in 16 accumulators, 4 head blocks x 4 dim blocks),
//     its operand read transposed from the token-major tile by ds_read_b64_tr_b8 as in the split form.
// The tiles are token-major with the 592-byte stride of the split form. The score reads are 128-bit, one per pair of
// MFMA steps (lane group q4 takes dims 64 j + 16 q4 .. + 15 of its row for steps 2 j, 2 j + 1; the query operand
// uses the same dim order): LDS serves them 8 lanes at a time, and 8 rows at one column cover the 32 banks once at
// the 592-byte stride (148 dwords, 4 mod 8). An odd last step (576-wide rows) reads 64 bits.
// Slot forms: token (idx + cnt + table, with the pooled variant of PoolForm) and rows + cnt; no bias array.
constexpr int AW_HEADS = 64;
constexpr int AW_MAXSLOTS = 33 * ATT_CH;  // 2,112: keep 2,048 plus a pooled tail
constexpr float AW_SLACK = 8.0f;          // lazy rescaling: p = exp(s - m) <= e^8 between moves of m

struct AttWideShared {
  uint8_t kt[2][ATT_CHUNK_BYTES];  // token-major e4m3 rows of two chunks (the queries before them)
  uint16_t p[AW_HEADS * ATT_PROW];  // bf16 P[head][token] of the current chunk
  int slot[AW_MAXSLOTS];
  float kscale[AW_MAXSLOTS];  // the slots' kv scales (the P weights' dequantisation)
  float kfac[AW_MAXSLOTS];    // kv scale x softmax scale (the scores' factor)
  float bias[AW_MAXSLOTS];    // 0 live, NEG_INF masked (below n_eff), -inf past n_eff
  f32x4 xs[2][4][4][WAVE];   // [th][hg][token block][lane]: partial scores over dims half th
  float al[AW_HEADS];        // the chunk's rescale factor per head
  int rfl[4];                // per head block: whether any of its 16 factors differs from 1
  float lsum[2][AW_HEADS];   // [th][head]: final sums
  float mfin[AW_HEADS];      // final maxima
};

// The many-row form's gather of one chunk into registers: LPT 16-byte pieces per thread, piece u = tid + 512 i of the
// chunk's 64 rows (row u / PIECES, piece u % PIECES); the store of those registers into a tile.
template <int DQK, int LPT>
__device__ __forceinline__ void wide_gload(const uint8_t* __restrict__ kv, const int* slots, int tid, u32x4 (&r)[LPT]) {
  constexpr int PIECES = DQK / 16, UNITS = ATT_CH * PIECES;
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int u = min(tid + ATT_THREADS * i, UNITS - 1);
    const int row = u / PIECES, pc = u - row * PIECES;
    r[i] = *reinterpret_cast<const u32x4*>(kv + (size_t)slots[row] * DQK + 16 * pc);
  }
}

template <int DQK, int LPT>
__device__ __forceinline__ void wide_lstore(uint8_t* tile, int tid, const u32x4 (&r)[LPT]) {
  constexpr int PIECES = DQK / 16, UNITS = ATT_CH * PIECES;
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int u = min(tid + ATT_THREADS * i, UNITS - 1);
    const int row = u / PIECES, pc = u - row * PIECES;
    *reinterpret_cast<u32x4*>(tile + row * ATT_KROW + 16 * pc) = r[i];
  }
}

template <int DQK>
__global__ __launch_bounds__(ATT_THREADS, 1) void sparse_mla_wide_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv, const float* __restrict__ kvs,
    const int* __restrict__ idx, const int* __restrict__ cnt, const int* __restrict__ table,
    const int* __restrict__ rows, uint16_t* __restrict__ out, float* __restrict__ out_f32,
    float* __restrict__ lse_out, int H, int keep, int max_pages, int page_size, int num_pages, float scale,
    PoolForm pf) {
  constexpr int PIECES = DQK / 16;                              // 16-byte data pieces per row
  constexpr int QROW = DQK + 8;                                 // staged query row stride (bf16 elements)
  constexpr int STEPS = DQK / 32;                               // score steps of 32 dims
  constexpr int UNITS = ATT_CH * PIECES;                        // 16-byte pieces per chunk
  constexpr int LPT = (UNITS + ATT_THREADS - 1) / ATT_THREADS;  // per thread and chunk: 5 or 4
  constexpr int QPIECES = AW_HEADS * DQK / 8;
  constexpr int QPT = (QPIECES + ATT_THREADS - 1) / ATT_THREADS;
  constexpr int SPT = (AW_MAXSLOTS + ATT_THREADS - 1) / ATT_THREADS;
  static_assert(AW_HEADS * QROW * 2 <= 2 * ATT_CHUNK_BYTES && STEPS % 2 == 0, "staging");
  __shared__ AttWideShared sh;
  const int HB = H / AW_HEADS;
  const int b = blockIdx.x / HB, hb64 = blockIdx.x - b * HB;
  if (pf.n_live && b >= *pf.n_live) return;  // a row past the run-time live count: left unwritten
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int hg = wave & 3, th = wave >> 2;
  const int l16 = lane & 15, q4 = lane >> 4;
  const bool token_form = rows == nullptr;

  // live slots (as in the split form): cnt_b of keep, at least one (a row with none attends slot 0 fully masked)
  int cnt_b = cnt[b];
  int pools_b = 0, tail_pool = 0;
  if (pf.kp_shift) {
    pools_b = min(max(cnt_b, 0), pf.idx_stride);
    tail_pool = max(pf.npool[b], 0);
    const int tail = min(max(pf.positions[b] + 1 - (tail_pool << pf.kp_shift), 0), (1 << pf.kp_shift) - 1);
    cnt_b = (pools_b << pf.kp_shift) + tail;
  }
  const int n_eff = cnt_b < 1 ? min(max(pf.empty_n, 1), keep) : (cnt_b > keep ? keep : cnt_b);
  const int nch = (n_eff + ATT_CH - 1) / ATT_CH;
  const int nslot = nch * ATT_CH;
  const size_t nslots_cache = (size_t)num_pages * page_size;

  // one round of loads: the 64 heads' queries, the slot ids of every chunk; then the slots' scales
  const u32x4* qsrc = reinterpret_cast<const u32x4*>(q + ((size_t)b * H + AW_HEADS * hb64) * DQK);
  u32x4 qv[QPT];
#pragma unroll
  for (int i = 0; i < QPT; ++i) qv[i] = qsrc[min(tid + ATT_THREADS * i, QPIECES - 1)];
  const int* trow = table ? table + (size_t)b * max_pages : nullptr;
  int slot_r[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int k = min(tid + ATT_THREADS * i, keep - 1);
    int slot;
    if (token_form) {
      int pos;
      if (pf.kp_shift) {
        const int j = k >> pf.kp_shift;
        const int pool = j < pools_b ? idx[(size_t)b * pf.idx_stride + j] : tail_pool;
        pos = (pool << pf.kp_shift) + (k & ((1 << pf.kp_shift) - 1));
      } else {
        pos = idx[(size_t)b * keep + k];
      }
      pos = pos < 0 ? 0 : pos;
      int pi = pos / page_size;
      pi = pi < max_pages ? pi : max_pages - 1;
      slot = safe_page(trow[pi], num_pages) * page_size + (pos - (pos / page_size) * page_size);
    } else {
      slot = rows[(size_t)b * keep + k];
      slot = ((size_t)(unsigned)slot < nslots_cache) ? slot : 0;
    }
    slot_r[i] = slot;
  }
  float ksc_r[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) ksc_r[i] = kvs ? kvs[slot_r[i]] : 1.0f;  // null: the unscaled cache
  uint16_t* qs = reinterpret_cast<uint16_t*>(&sh.kt[0][0]);
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int pc = tid + ATT_THREADS * i;
    if (pc < QPIECES) *reinterpret_cast<u32x4*>(qs + (pc / (DQK / 8)) * QROW + 8 * (pc % (DQK / 8))) = qv[i];
  }
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int k = tid + ATT_THREADS * i;
    if (k < nslot) {
      sh.slot[k] = slot_r[i];
      sh.kscale[k] = ksc_r[i];
      sh.kfac[k] = ksc_r[i] * scale;
      sh.bias[k] = k < n_eff ? (k < cnt_b ? 0.0f : NEG_INF) : -INFINITY;
    }
  }
  __syncthreads();
  constexpr int S2 = STEPS / 2;  // score steps per dims half
  bf16x8 qb[S2];
  {
    // the key operand's dim order (below): steps 2 j, 2 j + 1 give lane group q4 dims 64 j + 16 q4 + 8 (st % 2) ..
    // + 7 of the wave's half; an odd last step dims 32 st + 8 q4 .. + 7
    const uint16_t* qh = qs + (16 * hg + l16) * QROW + 32 * S2 * th;
#pragma unroll
    for (int st = 0; st < S2; ++st) {
      const int d = st < (S2 & ~1) ? 64 * (st >> 1) + 16 * q4 + 8 * (st & 1) : 32 * st + 8 * q4;
      qb[st] = as_bf16x8(*reinterpret_cast<const uint4*>(qh + d));
    }
  }
  __syncthreads();  // every wave holds its operand before the tiles overwrite the queries

  f32x4 o[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) o[i][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // running max of head 16 hg + l16 (the same in both th waves)
  float l_run = 0.0f;       // this lane's share of the running sum of head 16 hg + l16

  // chunk c from tile buf (in LDS since the previous chunk's last barrier); rn holds the next chunk's rows, stored
  // into the other tile once every wave is past its reads of it, then reloaded with chunk c + 3
  auto compute = [&](int c, int buf, u32x4(&rn)[LPT]) __attribute__((always_inline)) {
    const uint8_t* kt = sh.kt[buf];
    const int cb = c * ATT_CH;
    // partial scores of the 64 tokens (block k: tokens 16 k + l16 as MFMA rows) over this wave's dims half; lane
    // (l16, q4) reads 16 bytes of its row per pair of steps (dims 64 j + 16 q4 ..: one ds_read_b128 for two MFMAs),
    // 8 lanes of one 16-byte column at the 592-byte row stride covering the 32 banks once
    const uint8_t* krow = kt + l16 * ATT_KROW + 32 * S2 * th;
    f32x4 acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < S2 / 2; ++j) {
      u32x4 kk[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) kk[k] = *reinterpret_cast<const u32x4*>(krow + 16 * k * ATT_KROW + 64 * j + 16 * q4);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[k][0], kk[k][1]), qb[2 * j], acc[k], 0, 0,
                                                         0);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[k][2], kk[k][3]), qb[2 * j + 1], acc[k],
                                                         0, 0, 0);
    }
    if (S2 & 1) {
      constexpr int st = S2 - 1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint2 ka = *reinterpret_cast<const uint2*>(krow + 16 * k * ATT_KROW + 32 * st + 8 * q4);
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(ka.x, ka.y), qb[st], acc[k], 0, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) sh.xs[th][hg][k][lane] = acc[k];
    __syncthreads();  // both halves' partial scores; every wave is past the previous chunk's value reads
    wide_lstore<DQK, LPT>(sh.kt[buf ^ 1], tid, rn);
    wide_gload<DQK, LPT>(kv, &sh.slot[min(c + 3, nch - 1) * ATT_CH], tid, rn);
    // acc[k][r] + the other half's = S^T[token 16 k + 4 q4 + r][head 16 hg + l16]
    float sv[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 o4 = sh.xs[th ^ 1][hg][k][lane];
      const float4 kf = *reinterpret_cast<const float4*>(&sh.kfac[cb + 16 * k + 4 * q4]);
      const float4 bs = *reinterpret_cast<const float4*>(&sh.bias[cb + 16 * k + 4 * q4]);
      sv[k][0] = fmaf(acc[k][0] + o4[0], kf.x, bs.x);
      sv[k][1] = fmaf(acc[k][1] + o4[1], kf.y, bs.y);
      sv[k][2] = fmaf(acc[k][2] + o4[2], kf.z, bs.z);
      sv[k][3] = fmaf(acc[k][3] + o4[3], kf.w, bs.w);
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = max_nonan(mx, sv[k][r]);
    }
    mx = max_nonan(mx, __shfl_xor(mx, 16, WAVE));
    mx = max_nonan(mx, __shfl_xor(mx, 32, WAVE));
    // lazy rescaling: the running maximum moves only when the chunk's exceeds it by more than AW_SLACK, so most
    // chunks rescale nothing; p = exp(s - m) then stays below e^AW_SLACK, and o, l and lse use the same m (exact)
    const bool move = mx > m_run + AW_SLACK;
    const float m_new = move ? mx : m_run;
    const float alpha = move ? __expf(m_run - m_new) : 1.0f;
    m_run = m_new;
    if (th == 0) {
      const bool any = __ballot(move) != 0;
      if (lane == 0) sh.rfl[hg] = any;
    }
    float psum = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // this wave's tokens: blocks 2 th, 2 th + 1
      uint32_t pk[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int tk = cb + 32 * th + 16 * k + 4 * q4 + r;
        const float s0 = th ? sv[2 + k][r] : sv[k][r], s1 = th ? sv[2 + k][r + 1] : sv[k][r + 1];
        const float p0 = __expf(s0 - m_new), p1 = __expf(s1 - m_new);
        psum += p0 + p1;
        pk[r / 2] = bf16_pack(p0 * sh.kscale[tk], p1 * sh.kscale[tk + 1]);
      }
      *reinterpret_cast<uint2*>(&sh.p[(16 * hg + l16) * ATT_PROW + 32 * th + 16 * k + 4 * q4]) =
          make_uint2(pk[0], pk[1]);
    }
    l_run = l_run * alpha + psum;
    if (th == 0 && lane < 16) sh.al[16 * hg + lane] = alpha;
    __syncthreads();  // P and the rescale factors, and the next chunk's tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (sh.rfl[i]) {  // the same for every lane: a head block with no moved maximum is skipped
        const float4 a4 = *reinterpret_cast<const float4*>(&sh.al[16 * i + 4 * q4]);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          o[i][n][0] *= a4.x;
          o[i][n][1] *= a4.y;
          o[i][n][2] *= a4.z;
          o[i][n][3] *= a4.w;
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 pop[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pop[i] = as_bf16x8(*reinterpret_cast<const uint4*>(&sh.p[(16 * i + l16) * ATT_PROW + 32 * ks + 8 * q4]));
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const bf16x8 v = value_operand(kt, ks, 4 * wave + n, lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[i], v, o[i][n], 0, 0, 0);
      }
    }
    // the next chunk's partial scores, P and factors are written after its first barrier, which every wave reaches
    // only after this chunk's P . V
  };

  // the pipeline: chunk c computes from tile c % 2 and, between its two barriers, stores chunk c + 1 (loaded two
  // chunks earlier) into the other tile and reuses those registers for chunk c + 3; two barriers per chunk
  // (past the last chunk the loads re-read the last chunk, so every load is unconditional and the waits stay exact)
  u32x4 r0[LPT], r1[LPT];
  wide_gload<DQK, LPT>(kv, &sh.slot[0], tid, r0);
  wide_gload<DQK, LPT>(kv, &sh.slot[min(1, nch - 1) * ATT_CH], tid, r1);
  wide_lstore<DQK, LPT>(sh.kt[0], tid, r0);
  wide_gload<DQK, LPT>(kv, &sh.slot[min(2, nch - 1) * ATT_CH], tid, r0);
  __syncthreads();  // tile 0 in LDS
  for (int c = 0; c < nch; c += 2) {
    compute(c, 0, r1);
    if (c + 1 < nch) compute(c + 1, 1, r0);  // workgroup-uniform
  }

  // per head: the sum over both token halves, the final max
  float lw = l_run;
  lw += __shfl_xor(lw, 16, WAVE);
  lw += __shfl_xor(lw, 32, WAVE);
  if (lane < 16) {
    sh.lsum[th][16 * hg + lane] = lw;
    if (th == 0) sh.mfin[16 * hg + lane] = m_run;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = 16 * i + 4 * q4 + r;
      const float l = sh.lsum[0][head] + sh.lsum[1][head];
      const float inv = 1.0f / l;
      const size_t ob = ((size_t)b * H + AW_HEADS * hb64 + head) * ATT_DV + 64 * wave + l16;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float v = o[i][n][r] * inv;
        if (out) out[ob + 16 * n] = f32_to_bf16_bits(v);
        if (out_f32) out_f32[ob + 16 * n] = v;
      }
      if (lse_out && wave == 0 && l16 == 0)
        lse_out[(size_t)b * H + AW_HEADS * hb64 + head] = sh.mfin[head] + __logf(l);
    }
}

// o = sum_s W_s o_s / sum_s W_s with W_s = l_s exp(m_s - M), M = max_s m_s, and lse = M + log sum_s W_s, per
// (sequence, head), from each split's normalised o_s, max m_s and sum l_s (the log-sum-exp combine of
// trnrt/models/mla.py:853-856 with lse_s = m_s + log l_s kept in two parts); 128 threads x 4 dims. Every load is
// issued before any is used (one memory round trip; unconditional, so the waits count exactly); an empty split's
// o_s is 0 and its weight 0.
template <int S>
__global__ __launch_bounds__(128) void combine_splits_kernel(const float* __restrict__ ws_o,
                                                             const float* __restrict__ ws_ml, int H, int splits,
                                                             uint16_t* __restrict__ out, float* __restrict__ out_f32,
                                                             float* __restrict__ lse_out,
                                                             const int* __restrict__ n_live) {
  const int bh = blockIdx.x;
  const int b = bh / H, head = bh - b * H;
  if (n_live && b >= *n_live) return;  // a row past the run-time live count: left unwritten
  const int d = 4 * threadIdx.x;
  float2 ml[S];
  float4 v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const size_t i = ((size_t)b * splits + min(s, splits - 1)) * H + head;
    ml[s] = *reinterpret_cast<const float2*>(&ws_ml[2 * i]);
    v[s] = *reinterpret_cast<const float4*>(&ws_o[i * ATT_DV + d]);
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < S; ++s) M = s < splits ? fmaxf(M, ml[s].x) : M;
  float W = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float wt = (s < splits && ml[s].y > 0.0f) ? ml[s].y * __expf(ml[s].x - M) : 0.0f;
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
  if (out_f32)
    *reinterpret_cast<float4*>(&out_f32[oi]) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
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

// The attention's slots of query n (the arithmetic of trnrt/models/dsa_long.py:189-215 `slots` for any kpool kp):
// slot s < keep the selected pool pools[n, s] (taken when s < cnt[n]), slot keep the query's tail pool npool[n]
// (its tokens kp npool .. positions[n]), the rest pool 0 (masked); rows = the pool's row of the latent cache viewed
// as [slots / kp, kp R] through the query's table, bias 0 for every token to attend and NEG_INF otherwise.
__global__ void pool_slots_kernel(const int* __restrict__ pools, const int* __restrict__ cnt,
                                  const int* __restrict__ npool, const int* __restrict__ positions,
                                  const int* __restrict__ table, int table_shared, int* __restrict__ rows,
                                  float* __restrict__ bias, int keep, int n_slots, int table_pages, int ppp, int kp) {
  const int n = blockIdx.y;
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= n_slots) return;
  const int last_pool = table_pages * ppp - 1;
  const int np = npool[n];
  int pl = s < keep ? pools[(size_t)n * keep + s] : (s == keep ? min(np, last_pool) : 0);
  pl = min(max(pl, 0), last_pool);  // in range whatever the inputs
  const int pg = pl / ppp;
  const int* tab = table + (table_shared ? 0 : (size_t)n * table_pages);
  rows[(size_t)n * n_slots + s] = tab[pg] * ppp + (pl - pg * ppp);
  const bool sel_ok = s < keep && s < cnt[n];
  const int pos = positions[n];
  for (int t = 0; t < kp; ++t) {
    const bool tail_ok = s == keep && (long)np * kp + t <= (long)pos;
    bias[((size_t)n * n_slots + s) * kp + t] = (sel_ok || tail_ok) ? 0.0f : NEG_INF;
  }
}

hipError_t launch_pool_slots(const int* pools, const int* cnt, const int* npool, const int* positions,
                             const int* table, int table_shared, int* rows, float* bias, int N, int keep, int n_slots,
                             int table_pages, int page_size, int kp, hipStream_t s) {
  return launch("pool_slots_kernel", pool_slots_kernel, dim3((n_slots + 255) / 256, N), dim3(256), s, pools, cnt,
                npool, positions, table, table_shared, rows, bias, keep, n_slots, table_pages, page_size / kp, kp);
}

// Whether a launch of one split takes the many-row form: 64-head workgroups, the token form or rows + cnt (no bias
// array), at most AW_MAXSLOTS slots, and at least one workgroup per CU.
bool attention_wide_ok(int B, int H, int keep, bool has_bias, int num_cu) {
  return H % AW_HEADS == 0 && keep <= AW_MAXSLOTS && !has_bias && (long)B * (H / AW_HEADS) >= num_cu;
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

// keep: slots per row; in the pooled form (pf.kp_shift > 0) kpool x pf.idx_stride, the selected pools' tokens, with
// the row's tail tokens on top.
hipError_t launch_sparse_mla(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* idx, const int* cnt,
                             const int* table, const int* rows, const float* bias, uint16_t* out, float* out_f32,
                             float* lse, void* ws, int B, int H, int Dqk, int keep, int max_pages, int page_size,
                             int num_pages, float scale, int splits, hipStream_t s, PoolForm pf, bool wide) {
  if (splits == 1 && wide) {
    // the many-row form takes the pooled tail among its slots: kpool more
    const int keep_w = pf.kp_shift ? keep + (1 << pf.kp_shift) : keep;
    pf.tail_apart = 0;
    const dim3 grid(B * (H / AW_HEADS));
    return Dqk == 512 ? launch("sparse_mla_wide_kernel", sparse_mla_wide_kernel<512>, grid, dim3(ATT_THREADS), s, q,
                               kv, kvs, idx, cnt, table, rows, out, out_f32, lse, H, keep_w, max_pages, page_size,
                               num_pages, scale, pf)
                      : launch("sparse_mla_wide_kernel", sparse_mla_wide_kernel<576>, grid, dim3(ATT_THREADS), s, q,
                               kv, kvs, idx, cnt, table, rows, out, out_f32, lse, H, keep_w, max_pages, page_size,
                               num_pages, scale, pf);
  }
  // the split form adds the pooled tail apart from its keep slots when its rows fit their LDS (kpool 8 with 576-wide
  // rows: 7 x 576 bytes do not; the tail is then among the slots, keep + kpool of them)
  pf.tail_apart = pf.kp_shift && ((1 << pf.kp_shift) - 1) * Dqk <= ATT_TAIL_BYTES;
  if (pf.kp_shift && !pf.tail_apart) keep += 1 << pf.kp_shift;
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
  hipError_t e =
      Dqk == 512
          ? launch("sparse_mla_kernel", sparse_mla_kernel<512>, dim3(grid), dim3(ATT_THREADS), s, q, kv, kvs, idx, cnt,
                   table, rows, bias, out, out_f32, lse, ws_o, ws_ml, B, H, keep, max_pages, page_size, num_pages,
                   scale, eff_splits, sps, pf)
          : launch("sparse_mla_kernel", sparse_mla_kernel<576>, dim3(grid), dim3(ATT_THREADS), s, q, kv, kvs, idx, cnt,
                   table, rows, bias, out, out_f32, lse, ws_o, ws_ml, B, H, keep, max_pages, page_size, num_pages,
                   scale, eff_splits, sps, pf);
  if (e != hipSuccess || eff_splits == 1) return e;
  if (eff_splits <= 8)
    return launch("combine_splits_kernel", combine_splits_kernel<8>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H,
                  eff_splits, out, out_f32, lse, pf.n_live);
  if (eff_splits <= 16)
    return launch("combine_splits_kernel", combine_splits_kernel<16>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H,
                  eff_splits, out, out_f32, lse, pf.n_live);
  return launch("combine_splits_kernel", combine_splits_kernel<32>, dim3(B * H), dim3(128), s, ws_o, ws_ml, H,
                eff_splits, out, out_f32, lse, pf.n_live);
}

hipError_t launch_token_rows(const int* idx, const int* cnt, const int* table, int* rows, float* bias, int B,
                             int keep, int max_pages, int page_size, int num_pages, hipStream_t s) {
  launch("token_rows_kernel", token_rows_kernel, dim3((keep + 255) / 256, B), dim3(256), s, idx, cnt, table, rows, bias,
                     keep, max_pages, page_size, num_pages);
  return hipGetLastError();
}

}  // namespace dsa
