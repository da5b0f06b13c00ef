// Dense (prefill-chunk) lightning indexer for gfx950: the index scores of N queries that share one context's keys
// (the arithmetic of trnrt/kernels/dsa_long_select.py:119-133 `emulate_scores` and trnrt/models/dsa_long.py:74-84
// `scores` with a 2-D key tensor), with per-token FP8 key scales applied after the dot product:
//
//   score[n, p] = scale * k_scale[p] * sum_h w[n, h] * relu(q[n, h, :] . k_fp8[p, :])   for p < npool[n]
//   score[n, p] = NEG_INF                                                               for npool[n] <= p < stride
//
// (relu(a x) = a relu(x) for a = scale * k_scale[p] > 0, so this is dsa_long.scores' w relu(scale q . pk) with
// pk = k_fp8 k_scale.) It is a batched GEMM, (query, head) rows x keys over 128 dims, with a head-reducing epilogue.
// One workgroup = 4 queries (one per wave) x a block of keys, walked in tiles of 32: the workgroup loads a tile's
// 4 KiB of keys coalesced (16 bytes per thread), converts them once to bf16 (exact) into LDS, and every wave
// multiplies its query's 64 heads against them with v_mfma_f32_32x32x16_bf16 (heads as rows: the query operand
// stays in registers for the whole block), so each key byte is read from memory once per 4 queries and converted
// once per workgroup. The bf16 tile is double-buffered (one barrier per tile) and stored with an XOR swizzle (piece
// p of key j at slot 16 j + (p ^ (j & 15))) so the operand reads of 16 lanes hit 16 different bank groups.
//
// Every product is exact in the fp32 accumulator (bf16 x bf16), as in the reference's bf16 matmul; only the fp32
// summation order differs (the reference sums even and odd heads in two accumulators; this sums per lane, then
// across the two lane halves).
#include "dsa_common.h"

namespace dsa {

constexpr int PF_D = 128;
constexpr int PF_TILE = 32;                // keys per tile (one MFMA column block)
constexpr int PF_THREADS = 256;            // 4 waves, one query each
constexpr int PF_QPW = PF_THREADS / WAVE;  // queries per workgroup
constexpr int PF_TILES = 64;               // tiles per workgroup: 2048 keys
constexpr int PF_TPB = 4;                  // tiles per barrier (a "round": 128 keys)
constexpr int PF_RING = 2 * PF_TPB;        // tiles in flight per thread: two rounds ahead
constexpr int PF8_TPB = 2;                 // rounds of 64 keys (fewer registers and LDS: 3 workgroups a CU)
constexpr int PF8_RING = 2 * PF8_TPB;
static_assert(PF_TILES % PF8_RING == 0, "a block is whole ring turns");
static_assert(PF_TILES % PF_RING == 0, "a block is whole ring turns");

// MT: head tiles of 32 (Hi <= 32 MT).
// The two-level selection's sub-block maxima, taken by the workgroup that wrote the scores: after its last tile the
// wave of query n reads its row's scores of the block [p_begin, p_end) back (srow[p - base]: the FP8 form
// from its LDS copy of them, the bf16 form from the L2 after a barrier) and writes bm[n, b] = the maximum of the
// 2^sub_log2 scores of sub-block b, for b below nb. Scores past the candidates are NEG_INF, so this is the maximum
// over the candidates, as block_max_kernel computes it; vec: 16-byte aligned rows, read 16 bytes at a time where a
// sub-block holds a whole number of float4s (sub-blocks of 2 are read score by score: a float4 would take the next
// sub-block's two scores into this one's maximum).
__device__ __forceinline__ void block_max_rows(const float* srow, int base, float* __restrict__ bmrow, int p_begin,
                                               int p_end, int sub_log2, int nb, bool vec, int lane) {
  const int sub = 1 << sub_log2;
  const int b1 = min(nb, (p_end + sub - 1) >> sub_log2);
  vec = vec && sub >= 4;
  for (int b = (p_begin >> sub_log2) + lane; b < b1; b += WAVE) {
    const int p0 = b << sub_log2;
    float m = NEG_INF;
    if (vec && p0 + sub <= p_end) {
      for (int e = 0; e < sub; e += 4) {
        const float4 x = *reinterpret_cast<const float4*>(srow + (p0 + e - base));
        m = max_nonan(max_nonan(m, x.x), max_nonan(x.y, max_nonan(x.z, x.w)));
      }
    } else {
      for (int e = 0; e < sub && p0 + e < p_end; ++e) m = max_nonan(m, srow[p0 + e - base]);
    }
    bmrow[b] = m;
  }
}

// BF16K: the keys are bf16 [P, 128] with no per-key scale (GLM's pool keys, trnrt/models/dsa_long.py:74-84 over
// trnrt/models/mla.py:491-503 `context_pool_keys`): a thread's share of a tile is 32 bytes (two loads) that go to
// LDS as they are, so the ring holds twice the registers (taken at MT 1 only).
template <int MT, bool BF16K>
__global__ __launch_bounds__(PF_THREADS, MT == 1 ? 3 : 2) void indexer_prefill_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ w, const void* __restrict__ kcache_v,
    const float* __restrict__ kscale, const int* __restrict__ npool, float* __restrict__ scores, int N, int Hi, int P,
    int stride, float scale, float* __restrict__ bm, int sub_log2, int nb) {
  static_assert(!BF16K || MT == 1, "bf16 keys: up to 32 heads");
  // rounds of TPB tiles, RING in flight: at 32 heads rounds of 2 (fewer registers and LDS: 3 workgroups a CU), at 64
  // rounds of 4 (2 workgroups a CU; rounds of 2 there spill)
  constexpr int TPB = MT == 1 ? PF8_TPB : PF_TPB, RING = 2 * TPB;
  static_assert(PF_TILES % RING == 0, "a block is whole ring turns");
  const uint8_t* kcache = static_cast<const uint8_t*>(kcache_v);
  // two rounds of bf16 tiles (key j of a tile: 16 pieces of 8 dims, piece p at slot 16 j + (p ^ (j & 15))), the
  // block's per-key scales and the queries' candidate counts
  __shared__ u32x4 kb[2][TPB][PF_TILE * 16];
  __shared__ float ksc_s[PF_TILES * PF_TILE];
  __shared__ int lmax[PF_QPW];
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;  // key column of an MFMA tile / head row of the query operand
  const int h = lane >> 5;  // lane half: dims 16 s + 8 h .. + 7 at step s
  const int n = blockIdx.x * PF_QPW + wave;
  const int nq = min(n, N - 1);  // a wave past N computes a copy of the last query and stores nothing
  const int p_begin = blockIdx.y * PF_TILES * PF_TILE;
  const int p_end = min(p_begin + PF_TILES * PF_TILE, stride);
  const int ntiles = (p_end - p_begin + PF_TILE - 1) / PF_TILE;

  // this thread's share of a tile: key t / 8, bytes 16 (t % 8) .. + 15 (coalesced), converted into two pieces.
  // Tiles are prefetched RING ahead into a ring of registers that is never copied (a copy of a register whose
  // load is in flight waits for it): every loop turn below is unrolled, so each slot is a fixed register.
  const int tk = threadIdx.x >> 3, tp = threadIdx.x & 7;
  constexpr int KB = BF16K ? 2 * PF_D : PF_D;  // key row bytes
  auto load_tile = [&](int it, int half) {
    const int key = min(p_begin + it * PF_TILE + tk, P - 1);  // in range whatever the block
    return *reinterpret_cast<const u32x4*>(kcache + (size_t)key * KB + (BF16K ? 32 * tp + 16 * half : 16 * tp));
  };
  u32x4 ring[RING], ring2[BF16K ? RING : 1];
#pragma unroll
  for (int u = 0; u < RING; ++u) {
    ring[u] = load_tile(u, 0);
    if (BF16K) ring2[u] = load_tile(u, 1);
  }
#pragma unroll
  for (int i = 0; i < PF_TILES * PF_TILE / PF_THREADS; ++i) {
    const int k = i * PF_THREADS + threadIdx.x;
    ksc_s[k] = BF16K ? 1.0f : kscale[min(p_begin + k, P - 1)];
  }

  int L = min(max(npool[nq], 0), P);
  if (lane == 0) lmax[wave] = L;

  // the query operand (head 32m + j, dims 16 s + 8 h .. + 7 at step s; zero heads past Hi) and head weights in the
  // accumulator layout (register r of head tile m: head 32m + 8(r/4) + 4h + r%4)
  bf16x8 qa[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int head = 32 * m + j;
    const uint16_t* qp = q + ((size_t)nq * Hi + min(head, Hi - 1)) * PF_D + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 16 * s);
      qa[m][s] = as_bf16x8(head < Hi ? v : make_uint4(0, 0, 0, 0));
    }
  }
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int head = 32 * m + 8 * (r >> 2) + 4 * h + (r & 3);
      const float x = w[(size_t)nq * Hi + min(head, Hi - 1)];
      wr[m][r] = head < Hi ? x : 0.0f;
    }
  __syncthreads();
  const int wg_L = max(max(lmax[0], lmax[1]), max(lmax[2], lmax[3]));

  float* srow = scores + (size_t)n * stride;
  if (p_begin >= wg_L) {  // no query of the workgroup has a candidate in the block: no MFMA
    if (n < N) {
      for (int p = p_begin + lane; p < p_end; p += WAVE) srow[p] = NEG_INF;
      if (bm)
        for (int b = (p_begin >> sub_log2) + lane; b < nb && (b << sub_log2) < p_end; b += WAVE)
          bm[(size_t)n * nb + b] = NEG_INF;
    }
    return;
  }

  // The relu-weighted head sum of tile t - 1 (accumulators `prev`) runs between the MFMAs of tile t (into `cur`),
  // so the VALU work of one tile overlaps the matrix work of the next.
  auto epilogue_part = [&](float& part, const f32x16(&prev)[MT], int s) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int e = 2 * s; e < 2 * s + 2; ++e) part = fmaf(wr[m][e], relu(prev[m][e]), part);
  };
  auto finish = [&](float part, int t) {  // score of tile t's key j, stored by the lanes of half 0
    part += __shfl_xor(part, 32, WAVE);
    const int pos = p_begin + t * PF_TILE + j;
    const float v = pos < L ? part * (ksc_s[t * PF_TILE + j] * scale) : NEG_INF;
    if (n < N && h == 0 && pos < p_end) srow[pos] = v;
  };
  auto tile_mma = [&](const u32x4* tile, int t, f32x16(&cur)[MT], const f32x16(&prev)[MT]) {
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int pc = 2 * s + h;
      const bf16x8 kbv = __builtin_bit_cast(bf16x8, tile[16 * j + (pc ^ (j & 15))]);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        cur[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kbv, s == 0 ? f32x16{} : cur[m], 0, 0, 0);
      epilogue_part(part, prev, s);
    }
    if (t > 0) finish(part, t - 1);
  };
  f32x16 acc_a[MT], acc_b[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc_b[m] = f32x16{};
  // a round: convert the round's TPB tiles from their ring slots into LDS, refill the slots RING tiles ahead,
  // one barrier, then the round's tiles on MFMA (even tiles into acc_a, odd into acc_b). Whole ring turns are run
  // unconditionally (each slot then has the same loads in flight after it); tiles past the block's last tile load
  // clamped keys and store nothing (their positions are at or past p_end).
  auto round = [&](int t0, auto base) {
    constexpr int U0 = decltype(base)::value;
    u32x4(*tiles)[PF_TILE * 16] = kb[(t0 / TPB) & 1];
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
      const u32x4 r = ring[U0 + u];
      if (BF16K) {
        tiles[u][16 * tk + ((2 * tp) ^ (tk & 15))] = r;
        tiles[u][16 * tk + ((2 * tp + 1) ^ (tk & 15))] = ring2[U0 + u];
        ring2[U0 + u] = load_tile(t0 + u + RING, 1);
      } else {
        const bf16x8 lo = fp8x8_to_bf16x8(r[0], r[1]), hi = fp8x8_to_bf16x8(r[2], r[3]);
        tiles[u][16 * tk + ((2 * tp) ^ (tk & 15))] = __builtin_bit_cast(u32x4, lo);
        tiles[u][16 * tk + ((2 * tp + 1) ^ (tk & 15))] = __builtin_bit_cast(u32x4, hi);
      }
      ring[U0 + u] = load_tile(t0 + u + RING, 0);
    }
    __syncthreads();  // the round is in LDS; the other round's buffers are free (every wave finished them)
#pragma unroll
    for (int u = 0; u < TPB; u += 2) {
      tile_mma(tiles[u], t0 + u, acc_a, acc_b);
      tile_mma(tiles[u + 1], t0 + u + 1, acc_b, acc_a);
    }
  };
  int t = 0;
  for (; t < ntiles; t += RING) {
    round(t, std::integral_constant<int, 0>{});
    round(t + TPB, std::integral_constant<int, TPB>{});
  }
  float part = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) epilogue_part(part, acc_b, s);
  finish(part, t - 1);
  if (bm) {
    __syncthreads();  // the workgroup's scores are written
    if (n < N) block_max_rows(srow, 0, bm + (size_t)n * nb, p_begin, p_end, sub_log2, nb, (stride & 3) == 0, lane);
  }
}

// The FP8-query form: q is e4m3 with a per-(query, head) fp32 scale. Then every product q8 k8 is exact in the
// fp32 accumulator of the f8f6f4 MFMA (e4m3 x e4m3), and the query scale folds into the head weight
// (relu(a x) = a relu(x), a > 0):
//
//   score[n, p] = scale * k_scale[p] * sum_h (w[n, h] q_scale[n, h]) * relu(q8[n, h, :] . k8[p, :])
//
// Same workgroup shape and round structure as above, but the keys stay FP8 end to end: a tile is staged into LDS
// as raw bytes (16 B per thread, no conversion) and read by each wave as the B operand of
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales): 64 dims per MFMA, so 2 MFMAs per 32 heads x 32 keys instead of
// 8 bf16 ones. Lane (j, h) at step s holds dims 64 s + 32 h .. + 31 of its head (A) and of key j (B); the
// contraction only needs A and B to use the same lane/byte -> dim map. Key j's 16-byte piece p sits at LDS slot
// 8 j + (p ^ g(j)), g(j) = (j ^ (j >> 3)) & 7, so any 8 (or 16) consecutive lanes of a read hit different banks.
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;

__device__ __forceinline__ int pf8_slot(int key, int piece) { return 8 * key + (piece ^ ((key ^ (key >> 3)) & 7)); }

template <int MT>
__global__ __launch_bounds__(PF_THREADS, 3) void indexer_prefill_fp8_kernel(
    const uint8_t* __restrict__ q8, const float* __restrict__ qscale, const float* __restrict__ w,
    const uint8_t* __restrict__ kcache, const float* __restrict__ kscale, const int* __restrict__ npool,
    float* __restrict__ scores, int N, int Hi, int P, int stride, float scale, float* __restrict__ bm, int sub_log2,
    int nb) {
  __shared__ u32x4 kb[2][PF8_TPB][PF_TILE * 8];  // two rounds of FP8 tiles (key j: 8 pieces of 16 bytes)
  __shared__ float ksc_s[PF_TILES * PF_TILE];
  __shared__ int lmax[PF_QPW];
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int j = lane & 31;
  const int h = lane >> 5;
  const int n = blockIdx.x * PF_QPW + wave;
  const int nq = min(n, N - 1);
  const int p_begin = blockIdx.y * PF_TILES * PF_TILE;
  const int p_end = min(p_begin + PF_TILES * PF_TILE, stride);
  const int ntiles = (p_end - p_begin + PF_TILE - 1) / PF_TILE;

  const int tk = threadIdx.x >> 3, tp = threadIdx.x & 7;
  auto load_tile = [&](int it) {
    const int key = min(p_begin + it * PF_TILE + tk, P - 1);
    return *reinterpret_cast<const u32x4*>(kcache + (size_t)key * PF_D + 16 * tp);
  };
  u32x4 ring[PF8_RING];
#pragma unroll
  for (int u = 0; u < PF8_RING; ++u) ring[u] = load_tile(u);
#pragma unroll
  for (int i = 0; i < PF_TILES * PF_TILE / PF_THREADS; ++i) {
    const int k = i * PF_THREADS + threadIdx.x;
    ksc_s[k] = kscale[min(p_begin + k, P - 1)];
  }
  int L = min(max(npool[nq], 0), P);
  if (lane == 0) lmax[wave] = L;

  // A operand: head 32 m + j, dims 64 s + 32 h .. + 31 (zero heads past Hi); head weights times the query scales in
  // the accumulator layout (register r of head tile m: head 32 m + 8 (r / 4) + 4 h + r % 4)
  i32x8 qa[MT][2];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int head = 32 * m + j;
    const uint8_t* qp = q8 + ((size_t)nq * Hi + min(head, Hi - 1)) * PF_D + 32 * h;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(qp + 64 * s);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(qp + 64 * s + 16);
      const u32x4 z = {};
      const u32x4 a0 = head < Hi ? lo : z, a1 = head < Hi ? hi : z;
      qa[m][s] = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    }
  }
  float wr[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int head = 32 * m + 8 * (r >> 2) + 4 * h + (r & 3);
      const size_t o = (size_t)nq * Hi + min(head, Hi - 1);
      wr[m][r] = head < Hi ? w[o] * qscale[o] : 0.0f;
    }
  __syncthreads();
  const int wg_L = max(max(lmax[0], lmax[1]), max(lmax[2], lmax[3]));

  float* srow = scores + (size_t)n * stride;
  if (p_begin >= wg_L) {
    if (n < N) {
      for (int p = p_begin + lane; p < p_end; p += WAVE) srow[p] = NEG_INF;
      if (bm)
        for (int b = (p_begin >> sub_log2) + lane; b < nb && (b << sub_log2) < p_end; b += WAVE)
          bm[(size_t)n * nb + b] = NEG_INF;
    }
    return;
  }

  auto epilogue_part = [&](float& part, const f32x16(&prev)[MT], int s) {  // 8 of the 16 registers per step
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int e = 8 * s; e < 8 * s + 8; ++e) part = fmaf(wr[m][e], relu(prev[m][e]), part);
  };
  auto finish = [&](float part, int t) {
    part += __shfl_xor(part, 32, WAVE);
    const int pos = p_begin + t * PF_TILE + j;
    const float v = pos < L ? part * (ksc_s[t * PF_TILE + j] * scale) : NEG_INF;
    if (n < N && h == 0 && pos < p_end) srow[pos] = v;
  };
  auto tile_mma = [&](const u32x4* tile, int t, f32x16(&cur)[MT], const f32x16(&prev)[MT]) {
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 b0 = tile[pf8_slot(j, 4 * s + 2 * h)], b1 = tile[pf8_slot(j, 4 * s + 2 * h + 1)];
      const i32x8 kbv = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
#pragma unroll
      for (int m = 0; m < MT; ++m)
        cur[m] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[m][s], kbv, s == 0 ? f32x16{} : cur[m], 0, 0, 0,
                                                                 127, 0, 127);
      epilogue_part(part, prev, s);
    }
    if (t > 0) finish(part, t - 1);
  };
  f32x16 acc_a[MT], acc_b[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc_b[m] = f32x16{};
  auto round = [&](int t0, auto base) {
    constexpr int U0 = decltype(base)::value;
    u32x4(*tiles)[PF_TILE * 8] = kb[(t0 / PF8_TPB) & 1];
#pragma unroll
    for (int u = 0; u < PF8_TPB; ++u) {
      tiles[u][pf8_slot(tk, tp)] = ring[U0 + u];
      ring[U0 + u] = load_tile(t0 + u + PF8_RING);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PF8_TPB; u += 2) {
      tile_mma(tiles[u], t0 + u, acc_a, acc_b);
      tile_mma(tiles[u + 1], t0 + u + 1, acc_b, acc_a);
    }
  };
  int t = 0;
  for (; t < ntiles; t += PF8_RING) {
    round(t, std::integral_constant<int, 0>{});
    round(t + PF8_TPB, std::integral_constant<int, PF8_TPB>{});
  }
  float part = 0.0f;
#pragma unroll
  for (int s = 0; s < 2; ++s) epilogue_part(part, acc_b, s);
  finish(part, t - 1);
  if (bm) {
    __syncthreads();  // the workgroup's scores are written
    if (n < N) block_max_rows(srow, 0, bm + (size_t)n * nb, p_begin, p_end, sub_log2, nb, (stride & 3) == 0, lane);
  }
}

template <int MT, bool BF16K>
static hipError_t launch_prefill_mt(const uint16_t* q, const float* w, const void* k, const float* ks,
                                    const int* npool, float* scores, int N, int Hi, int P, int stride, float scale,
                                    float* bm, int sub_log2, int nb, hipStream_t s) {
  const dim3 grid((N + PF_QPW - 1) / PF_QPW, (stride + PF_TILES * PF_TILE - 1) / (PF_TILES * PF_TILE));
  return launch("indexer_prefill_kernel", indexer_prefill_kernel<MT, BF16K>, grid, dim3(PF_THREADS), s, q, w, k, ks,
                npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb);
}

// bm (or null): also the sub-block maxima of 2^sub_log2 scores, [N, nb].
hipError_t launch_indexer_prefill(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                  const int* npool, float* scores, int N, int Hi, int P, int stride, float scale,
                                  float* bm, int sub_log2, int nb, hipStream_t s) {
  if (Hi <= 32)
    return launch_prefill_mt<1, false>(q, w, k, ks, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb, s);
  return launch_prefill_mt<2, false>(q, w, k, ks, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb, s);
}

// bf16 keys without scales (Hi <= 32).
hipError_t launch_indexer_prefill_bf16k(const uint16_t* q, const float* w, const uint16_t* k, const int* npool,
                                        float* scores, int N, int Hi, int P, int stride, float scale, float* bm,
                                        int sub_log2, int nb, hipStream_t s) {
  if (Hi > 32) return hipErrorInvalidValue;
  return launch_prefill_mt<1, true>(q, w, k, nullptr, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb, s);
}

}  // namespace dsa

namespace dsa {

template <int MT>
static hipError_t launch_prefill_fp8_mt(const uint8_t* q8, const float* qs, const float* w, const uint8_t* k,
                                        const float* ks, const int* npool, float* scores, int N, int Hi, int P,
                                        int stride, float scale, float* bm, int sub_log2, int nb, hipStream_t s) {
  const dim3 grid((N + PF_QPW - 1) / PF_QPW, (stride + PF_TILES * PF_TILE - 1) / (PF_TILES * PF_TILE));
  return launch("indexer_prefill_fp8_kernel", indexer_prefill_fp8_kernel<MT>, grid, dim3(PF_THREADS), s, q8, qs, w, k,
                ks, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb);
}

hipError_t launch_indexer_prefill_fp8(const uint8_t* q8, const float* qs, const float* w, const uint8_t* k,
                                      const float* ks, const int* npool, float* scores, int N, int Hi, int P,
                                      int stride, float scale, float* bm, int sub_log2, int nb, hipStream_t s) {
  if (Hi <= 32)
    return launch_prefill_fp8_mt<1>(q8, qs, w, k, ks, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb, s);
  return launch_prefill_fp8_mt<2>(q8, qs, w, k, ks, npool, scores, N, Hi, P, stride, scale, bm, sub_log2, nb, s);
}

}  // namespace dsa
