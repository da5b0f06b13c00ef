// The whole DSA decode layer step in one launch (trnrt/models/mla.py:506-528 `attention_long` at kpool 1: indexer ->
// exact top-keep -> sparse MLA; the single-call decode layer of trnrt/kernels/dsa_shell.py:2114-2321), for rows of up
// to 32,768 tokens.
//
// gfx950 has 8 XCDs of 32 CUs, each XCD with its own L2; workgroup x of a launch runs on XCD x % 8. Row b is owned by
// the 32 workgroups of XCD b % 8 (one per CU; a batch of more than 8 rows takes one launch per 8 rows), so every
// hand-off between the stages of a row stays inside one L2: a workgroup's stores are complete in that L2 once its
// memory counter drains, and its peers read them with plain loads, which miss their CU's L1 (nothing there holds
// those lines yet) and hit the XCD's L2. The stages are separated by XCD-local barriers on a counter word per XCD (an arrival is one atomic add; a
// waiter polls with sc1 loads, every wait bounded: past its limit the workgroup records an error flag and goes on, so
// no wave can hang).
//
// Per row of L tokens, workgroup j (of 32) owns positions kw j .. kw j + kw - 1, kw = 32 ceil(L / 1024) (1024 at
// most): the row's positions in 32 blocks of whole 32-key tiles, so every workgroup of a short row takes a share of
// its keys, and position order is workgroup order.
//   1. indexer: scores of the workgroup's positions (8 waves x up to 4 tiles of 32 keys, bf16 MFMA over the exactly
//      converted e4m3 keys, the weighted relu head sum in registers; the arithmetic of
//      trnrt/kernels/dsa_index.py:44-50), written to the scores output and kept in LDS, with an LDS histogram of the
//      top 12 bits of their order keys written as a list of its nonzero bins and, on most rows, a list of the
//      workgroup's largest keys (whole bins, at most 192, in position order); barrier A;
//   2+3 in one exchange (when every key at or above the row's keep-th largest is in the key lists, which the lists
//      themselves show): every workgroup reads the 32 key lists and finds T, the ties to take and each workgroup's
//      output offset from them alone, then lists its split's slots as stage 3 does; no barrier B. Otherwise:
//   2. selection, first level: the row histogram gives the bin c0 of the keep-th largest key; the workgroup counts its
//      keys above c0 and writes its keys in c0 (the candidates) in position order; barrier B;
//   3. selection, exact: every workgroup reads the row's candidates (a few hundred for indexer scores) and finds the
//      keep-th largest key T and the ties at T to take (the lowest positions, trnrt/models/dsa_select.py:10-38) by two
//      LDS histogram passes (12 + 8 bits), then each workgroup's count and offset in the ascending output; from the
//      row's bitmaps of selected positions the workgroup lists the cache slots of its own split's outputs and writes
//      their indices (no barrier before the attention);
//   4. attention: workgroup j takes head group j % (H / HPW) and split j / (H / HPW) of the ascending output: it
//      gathers its split's rows into LDS and computes softmax(scale q.K) V over the split in one pass (bf16 MFMA over
//      the exactly converted rows, fp32 softmax over the whole split), writing the split's output (the sum of
//      exp(score - max) v, divided in the combine) with its max and sum (the arithmetic of
//      trnrt/kernels/dsa_decode.py:26-37 and trnrt/kernels/dsa_slots.py:48-65);
//      barrier C;
//   5. combine: the splits merged by log-sum-exp (trnrt/models/mla.py:853-856), workgroup j for 1/32 of the outputs.
// The last workgroup of an XCD to finish resets the XCD's barrier words, so the workspace region that must be zero
// between calls is zero again.
#include "dsa_common.h"

namespace dsa {

constexpr int FU_XCDS = 8;
constexpr int FU_NW = 32;        // workgroups per XCD, one per CU
constexpr int FU_THREADS = 512;  // 8 waves: two per SIMD, so one's memory waits hide under the other's work
constexpr int FU_WAVES = FU_THREADS / WAVE;
constexpr int FU_TILE = 32;                           // keys per MFMA tile
constexpr int FU_TPW = 4;                             // tiles per wave
constexpr int FU_AHEAD = 2;                           // key tiles in flight ahead of the one a wave computes
constexpr int FU_KEYS = FU_WAVES * FU_TPW * FU_TILE;  // 1024: positions per workgroup at most (fu_kw)
constexpr int FU_MAXLEN = FU_NW * FU_KEYS;            // 32,768
constexpr int FU_D = 128;                             // indexer head dim
constexpr int FU_QROW = FU_D + 8;                     // staged indexer query row (bf16)
constexpr int FU_HBINS = HIST_BINS;
constexpr int FU_BUF_WORD3 = 0x00020000;  // buffer descriptor word 3 of raw dword loads (gfx9)
constexpr int FU_BMW = FU_KEYS / 32;    // words of a workgroup's bitmap of positions
// A workgroup's bin list: its count of nonzero histogram bins, then (bin << 16) | count for each
constexpr int FU_HROW = 1056;
constexpr int FU_HSTAGE = 256;  // words of each list every workgroup reads into LDS (the rest: read from the L2)
static_assert(FU_HROW >= 1 + FU_KEYS && FU_HROW % 4 == 0, "bin list");
// A workgroup's candidate block: its counts word, the bitmap of its keys above the first-level bin, its candidates
constexpr int FU_CROW = 1088;
constexpr int FU_CSTAGE = 128;                      // words of each block every workgroup reads into LDS
constexpr int FU_CSTAGED = FU_CSTAGE - 1 - FU_BMW;  // candidates among them (the rest: read from the L2)
static_assert(FU_CROW >= 1 + FU_BMW + FU_KEYS && FU_CROW % 4 == 0, "candidate block");
// A workgroup's key list: its visible keys in the histogram bins down to the one holding its FU_LM-th largest key (all
// of them when they number at most FU_LCAP; the bins above that one when it would hold more), in position order:
// a 128-byte header (count, lowest bin listed (0: every visible key), 0, 0, then the workgroup's FU_LBINS highest
// nonzero histogram bins as (bin << 16) | count in descending bin order, 0 past its nonzero bins), then (key,
// position in the workgroup's block) pairs. Read back by 16 threads of FU_LPT entries each. Rows whose blocks hold at
// most FU_LCAP positions (every list holds all its keys), or whose workgroups select FU_LM * 5 / 8 keys or fewer on
// average (at keep 2048: every row length), take the one-exchange selection from the lists; the others, and any row
// whose lists turn out not to hold its selection, the two-exchange form (stages 2 and 3).
constexpr int FU_LM = 128;
constexpr int FU_LPT = 12;
constexpr int FU_LCAP = 16 * FU_LPT;
constexpr int FU_LHDR = 32;                 // header words
constexpr int FU_LBINS = FU_LHDR - 4;       // bins in the header
constexpr int FU_LROW = FU_LHDR + 2 * FU_LCAP;
static_assert(FU_LBINS == 28, "two header bins for each of 14 of a list's 16 threads");
static_assert(FU_LM <= FU_LCAP && FU_LPT % 2 == 0, "key list");
// The layer's two forms: kpool 1 (FP8 keys with per-token scales; a workgroup's key list reaches down to the bin of
// its FU_LM-th largest key) and pooled (GLM's kpool > 1: the scores of bf16 pool keys with no scale, rows of at most
// 8,192 pools, so blocks of at most 256, every one of which its workgroup's list holds: the one-exchange selection
// always applies). A pooled list is the block's keys in position order, one word each (0: not selectable), then
// the block's FU_PBINS highest nonzero histogram bins as (bin << 16) | count in descending bin order (0 past its
// nonzero bins).
constexpr int FU_PBINS = 64;
template <bool POOL>
struct FuForm {
  static constexpr int LPT = POOL ? 16 : FU_LPT;  // list entries per reading thread
  static constexpr int LCAP = 16 * LPT;
  static constexpr int LROW = POOL ? LCAP + FU_PBINS : FU_LHDR + 2 * LCAP;
  static constexpr int KV = POOL ? 8 : 4;       // 16-byte key loads per lane and tile (64 bf16 or 64 e4m3 dims)
  static constexpr int TILE_LOADS = POOL ? 8 : 5;  // load instructions per lane and tile (with the scale)
  static_assert(LROW % 32 == 0 && LPT % 2 == 0, "key list");
};
constexpr int FU_POOL_MAXLEN = FU_NW * FuForm<true>::LCAP;  // 8,192 pools
static_assert(FU_HROW % 32 == 0 && FU_CROW % 32 == 0 && FU_LROW % 32 == 0, "a workgroup's rows in lines of its own");
constexpr int FU_CH = 64;          // slot granularity of a split
constexpr int FU_DQK = 576, FU_DV = 512;
constexpr int FU_PIECES = FU_DQK / 16;  // 36 16-byte pieces per row
constexpr int FU_KPIECES = FU_PIECES + 1;  // a staged row: the data and one padding piece (592 bytes), the stride at
                                           // which the operand reads of 8 or 16 rows at one column hit distinct banks
constexpr int FU_KROW = 16 * FU_KPIECES;
constexpr int FU_STEPS = FU_DQK / 32;   // score steps
constexpr int FU_AQROW = FU_DQK + 8;    // staged attention query row (bf16)
constexpr unsigned FU_SPIN = 1u << 20;  // polls before a wait gives up (a normal wait takes a few)

// LDS (160 KiB, one workgroup per CU), phase by phase:
constexpr int L_STATE = 0;       // FuState: selection results (stage 3)
constexpr int L_CO0 = 512;       // the one-exchange selection: coarse bins of its first level [64]
constexpr int L_CO1 = 768;       // and of its second [64]
constexpr int L_MISC = 1536;     // block-scan scratch (stages 1-3)
constexpr int L_HLS = 2048;      // stage 2: the first 256 words of every bin list [32][256]
constexpr int L_BINS2 = 2048;    // stage 3: 256 bins
constexpr int L_SPG = 12288;     // stage 3: the pages of the source positions [1024]
constexpr int L_CB = 16384;      // stage 3: the first 128 words of every candidate block [32][128]
constexpr int L_SB = 32768;      // stage 3: per workgroup the bitmap of its selected positions [32][32]
constexpr int L_PB = 36864;      // stage 3: their exclusive prefix popcounts [32][32]
constexpr int L_BINS = 40960;    // stage 3: 4096 bins
constexpr int L_QS = 32768;      // stage 1: indexer queries [64][136] bf16
constexpr int L_WS = 50176;      // stage 1: head weights [64]
constexpr int L_HS = 50432;      // stage 1: histogram [4096]
constexpr int L_HSC = 66816;     // stage 1: its coarse bins [64] (bins 64 c .. 64 c + 63)
constexpr int L_SCS = 159744;    // stages 1-3: the scores of the workgroup's 1024 positions (NEG_INF past its block)
constexpr int L_KT = 0;          // stage 4: the rows, token-major at the 592-byte stride
constexpr int FU_LDS = 163840;
static_assert(L_HS + 4 * FU_HBINS <= L_HSC && L_HSC + 4 * 64 <= L_SCS && FU_HBINS == 4096, "stage 1 layout");
static_assert(L_HLS + 4 * FU_NW * FU_HSTAGE <= L_HS, "stage 2 layout");
static_assert(L_BINS2 + 4 * 256 <= L_SPG && L_BINS + 4 * 4096 <= 57344, "stage 3 layout");
static_assert(L_SPG + 4 * 1024 <= L_CB && L_CB + 4 * FU_NW * FU_CSTAGE <= L_SB && L_SB + 4 * FU_NW * FU_BMW <= L_PB &&
                  L_PB + 4 * FU_NW * FU_BMW <= L_BINS,
              "stage 3 blocks");
static_assert(L_SCS + 4 * FU_KEYS == FU_LDS, "LDS size");

// The attention's shape: HPW heads per workgroup (16 or 32) over splits of up to 4096 / HPW slots of DQK-byte rows
// (576, or 512: GLM's NoPE latent), its 8 waves as TG groups of 32 tokens x HB blocks of 16 heads in the scores; with
// XT (the pooled form) a split holds up to 64 rows more (a pooled row's tail, padded), the waves of groups 0 and 1
// taking groups TG and TG + 1 as well. Its LDS past the gathered rows (CAP rows at the stride KROW): the split's slot
// list (later P [HPW][CAP + 8] bf16), kv scales and biases [CAP], per-wave head maxima and sums [HPW][TG], and (read
// before the gather) the HPW heads' queries [HPW][DQK + 8] bf16. A split's rows are padded to a multiple of FU_CH =
// 64: the gather's loads of 64 lanes x 16 bytes then cover its padded rows' pieces exactly (no lane of the last load
// reads a slot past the padded rows).
template <int HPW, int DQK = FU_DQK, bool XT = false>
struct FuAtt {
  static constexpr int SPLIT = 4096 / HPW;
  static constexpr int CAP = SPLIT + (XT ? FU_CH : 0);
  static constexpr int HB = HPW / 16;
  static constexpr int TG = SPLIT / 32;
  static constexpr int PROW = CAP + 8;
  static constexpr int PIECES = DQK / 16;        // 16-byte pieces of a row
  static constexpr int KPIECES = PIECES + 1;     // a staged row: its pieces and one padding piece
  static constexpr int KROW = 16 * KPIECES;      // 592 or 528 bytes: 8 rows at one column cover the banks once
  static constexpr int STEPS = DQK / 32;         // score steps
  static constexpr int AQROW = DQK + 8;          // staged query row (bf16)
  static constexpr int QPT = (HPW * DQK / 8 + FU_THREADS - 1) / FU_THREADS;  // query loads per thread
  static constexpr int L_P = CAP * KROW;
  static constexpr int L_KSC = L_P + 2 * HPW * PROW;
  static constexpr int L_BIAS = L_KSC + 4 * CAP;
  static constexpr int L_RED = L_BIAS + 4 * CAP;
  static constexpr int L_SRED = L_RED + 4 * TG * HPW;
  static constexpr int L_END = L_SRED + 4 * TG * HPW;
  static constexpr int L_QST = HPW == 16 ? 57344 : L_END;  // inside the row tile (read before the gather), or past it
};
static_assert(FuAtt<16>::TG * FuAtt<16>::HB == FU_WAVES && FuAtt<32>::TG * FuAtt<32>::HB == FU_WAVES, "waves");
static_assert(FuAtt<16>::L_END <= FU_LDS && FuAtt<16>::L_QST + 2 * 16 * FU_AQROW <= FuAtt<16>::L_P, "stage 4, 16");
static_assert(FuAtt<32>::L_QST + 2 * 32 * FU_AQROW <= L_SCS && FuAtt<32>::L_P >= 57344, "stage 4, 32");
static_assert(FuAtt<32, 512, true>::L_QST + 2 * 32 * FuAtt<32, 512, true>::AQROW <= FU_LDS &&
                  4 * FuAtt<32, 512, true>::CAP <= 2 * 32 * FuAtt<32, 512, true>::PROW,
              "the pooled form's attention");
static_assert(FuAtt<32>::KROW == FU_KROW && FuAtt<32>::STEPS == FU_STEPS && FuAtt<32>::AQROW == FU_AQROW, "shape");

struct FuState {
  int gt[FU_NW];  // per workgroup: its candidates above T
  int eq[FU_NW];  // its candidates equal to T
  int c0, above0, nvis, pad;
  int lbin[FU_NW];  // per workgroup: the lowest bin its key list holds
};
static_assert(sizeof(FuState) <= L_CO0 && L_CO1 + 4 * 64 <= L_MISC, "state");

struct FusedArgs {
  const uint16_t* q_idx;
  const float* w;
  const uint8_t* k;
  const float* ks;
  const uint16_t* q;
  const uint8_t* kv;
  const float* kvs;
  const int* table;
  const int* ctx_len;
  float* scores;
  int* idx;
  int* cnt;
  uint16_t* out;
  float* lse;
  uint32_t* hl;    // [B][32][1056]: per workgroup its histogram's nonzero bins (count, then (bin << 16) | count)
  int* sync;       // [8][16] at the workspace's start: per XCD the barrier arrivals and exits (zero between calls),
                   // the count of waits that gave up and of rows that took the two-exchange selection (kept until
                   // dsa_layer_status clears them)
  uint32_t* cand;  // [B][32][1088]: per workgroup (keys above c0) << 16 | (candidates), the bitmap of its positions
                   // above c0 (32 words), then the candidates, (low 20 key bits << 10) | position in the workgroup's
                   // range, in position order
  uint32_t* lst;   // [B][32][FuForm::LROW]: per workgroup its key list
  uint16_t* part;  // [B][S][H][512]: split outputs (bf16, sums of exp(score - split max) v), heads side by side

  float2* ml;      // [B][S][H]: split max and sum
  int B, Hi, H, max_pages, page_size, page_shift, num_pages, stride, keep;
  int num_slots;  // num_pages * page_size
  float scale;
  int HG, S, sps;
  // the pooled form of the separate attention launch (kp_shift > 0): idx holds [B][keep >> kp_shift] selected pools,
  // cnt their count, npool and positions the rows' complete pools and positions (the tail)
  const int* npool;
  const int* positions;
  int kp_shift;
  int ppp_shift;  // the pooled one-launch layer: log2 of the pools per page (pool p's key: page row p >> ppp_shift)
  // the pooled step (the pool-key write in the same launch): the indexer rows cache [slots][pk_width] (e4m3 with
  // pk_scale per slot, or bf16), the pool-position bias [kpool][128] and each row's written token's slot
  const void* pk_rows;
  const float* pk_scale;
  const float* pk_ape;
  const int64_t* slot_mapping;
  int pk_width, pk_fp8;
  int row0;  // this launch's first row (rows row0 .. row0 + 7)
};

// Device-scope loads (sc1) miss the CU's caches and are served past the XCD's L2 (measured: at a small fraction of
// the L2's bandwidth). The kernel uses them only for the barrier polls. Everything a peer publishes before a barrier
// (bin lists, candidate blocks, key lists, split outputs and their (max, sum) pairs) is read with plain loads, which
// hit the XCD's L2: a CU's L1 holds no stale copy of it, since the L1 is invalidated at each launch's start, no
// workgroup reads a peer's region before the barrier that publishes it, and each workgroup's region of each kind
// occupies whole 128-byte lines of its own.
constexpr int FU_AUX_PLAIN = 0;  // the cache-policy operand of the loads of a peer's published data: none

// XCD-local barrier of the 32 workgroups of an XCD: every thread's stores complete (drained memory counter), then the
// workgroup's arrival (one atomic add to each of the counter's WS_SYNC_LINES copies, a line each) and a bounded poll
// (atomic adds of 0) of copy j mod WS_SYNC_LINES. Each copy of the XCD's counter only grows: every launch adds exactly
// FU_SPAN = 8 x 32 to it (each workgroup one arrival per barrier, and the rest of its 8 at its exit, with no wait), so
// at a launch's start it holds a multiple of FU_SPAN plus the arrivals at this launch's first barrier (fewer than 32:
// that barrier needs every workgroup's); the base read then, rounded down to FU_SPAN, places the n-th barrier at
// base + 32 n arrivals (unsigned, so the counter may wrap). Every kernel using these barriers takes at most 8. A wait
// that gives up (all 32 workgroups must be resident at once: another kernel holding CUs for the whole poll budget,
// a fraction of a second, breaks that) counts itself in the XCD's status word and goes on; every read of a peer's data below
// stays inside its region whatever that data holds, so such a call ends normally, and dsa_layer_status reports it.
constexpr unsigned FU_SPAN = 8 * FU_NW;
struct FuSync {
  int* w;         // the XCD's words: the counter, then the status words
  unsigned* rep;  // the copy of the counter this workgroup polls
  unsigned base;  // the counter's value at this launch's start (thread 0's)
};

__device__ __forceinline__ FuSync fu_sync_begin(int* w, int j) {
  FuSync sy{w, reinterpret_cast<unsigned*>(w + WS_SYNC_LINE_WORDS * (j % WS_SYNC_LINES)), 0u};
  if (threadIdx.x == 0)
    sy.base = __hip_atomic_load(sy.rep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ~(FU_SPAN - 1u);
  return sy;
}

__device__ __forceinline__ void fu_barrier(const FuSync& sy, int n) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < WS_SYNC_LINES)  // the arrival, on every copy of the counter
    __hip_atomic_fetch_add(reinterpret_cast<unsigned*>(sy.w + WS_SYNC_LINE_WORDS * threadIdx.x), 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) {
    unsigned* ctr = sy.rep;
    const unsigned target = sy.base + (unsigned)n * FU_NW;
    unsigned polls = 0;
    // (each poll an atomic add of 0 with return, read where the arrivals are added: 0.57 us a launch faster than
    // device-scope loads; a literal 0 would be folded into such a load). Two polls are in flight, 512 clocks apart at
    // first, each reissued as soon as it returns short of the target; the address is passed through a VGPR, so the
    // compiler keeps each poll one atomic instruction and waits only for the older one (vmcnt(1)).
    unsigned z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    __attribute__((address_space(1))) unsigned* pc = (__attribute__((address_space(1))) unsigned*)ctr;
    asm volatile("" : "+v"(pc));
    unsigned p = __hip_atomic_fetch_add(pc, z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_sleep(8);
    unsigned q = __hip_atomic_fetch_add(pc, z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while ((int)(p - target) < 0) {
      if (++polls > FU_SPIN) {
        __hip_atomic_fetch_add(sy.w + WS_SYNC_GAVE_UP, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      p = q;
      q = __hip_atomic_fetch_add(pc, z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
}

// The workgroup's exit after nbar barriers: its remaining arrivals of the launch's FU_SPAN (one add, not waited for).
__device__ __forceinline__ void fu_exit(const FuSync& sy, int nbar) {
  if (threadIdx.x < WS_SYNC_LINES)
    __hip_atomic_fetch_add(reinterpret_cast<unsigned*>(sy.w + WS_SYNC_LINE_WORDS * threadIdx.x),
                           FU_SPAN / FU_NW - (unsigned)nbar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide over 512 threads, thread t holding the counts of bins PER t .. PER t + PER - 1 (higher bins = larger
// keys): the bin holding the need-th largest key and the keys in the bins above it; returns the total. scr: 16 ints
// of LDS, with scr[8] = -1 on entry (written before a barrier that precedes this call). Two barriers; the caller
// must pass one more before scr is written again. Counts that cannot hold the need-th key give bin 0, above 0.
template <int PER>
__device__ int fu_find_bin(const int (&hb)[PER], int need, int* scr, int* bin, int* above) {
  const int t = threadIdx.x, wave = t / WAVE, lane = t & (WAVE - 1);
  int mine = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) mine += hb[i];
  const int pre = wave_incl_scan(mine);
  const int inc = __builtin_amdgcn_readlane(pre, WAVE - 1) - pre + mine;  // inclusive suffix over the lanes
  if (lane == 0) scr[wave] = inc;
  __syncthreads();
  int after = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < FU_WAVES; ++w) {
    const int x = scr[w];
    after += w > wave ? x : 0;
    tot += x;
  }
  int excl = after + inc - mine;  // keys in the bins above this thread's
  if (excl < need && excl + mine >= need) {
#pragma unroll
    for (int i = PER - 1; i >= 0; --i) {
      if (excl < need) {
        if (excl + hb[i] >= need) {
          scr[8] = PER * t + i;
          scr[9] = excl;
        }
        excl += hb[i];
      }
    }
  }
  __syncthreads();
  const int b = scr[8];
  *bin = b < 0 ? 0 : b;
  *above = b < 0 ? 0 : scr[9];
  return tot;
}

// Wave-level (every wave alike, no barrier) over a 4096-bin histogram in LDS, fine[64 c + f], with its coarse bins
// coarse[c] = fine[64 c] + .. + fine[64 c + 63] (higher bins = larger keys): the bin holding the need-th largest key
// and the keys in the bins above it; returns the total. Lane l takes coarse bin l, then fine bin 64 k + l of the
// coarse bin k found (suffix sums over the lanes do not increase with the lane, so the lanes whose sum reaches need
// are lanes 0 .. k). Counts that cannot hold the need-th key (or need <= 0) give bin 0, above 0.
__device__ __forceinline__ int fu_wave_find(const int* fine, const int* coarse, int need, int* bin, int* above) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int cc = coarse[lane];
  const int pc = wave_incl_scan(cc);
  const int tot = __builtin_amdgcn_readlane(pc, WAVE - 1);
  const int sc = tot - pc + cc;  // coarse bins lane .. 63
  if (need <= 0 || tot < need) {  // wave-uniform
    *bin = 0;
    *above = 0;
    return tot;
  }
  const int k = __popcll(__ballot(sc >= need)) - 1;
  const int abv = __builtin_amdgcn_readlane(sc - cc, k);  // keys above coarse bin k
  const int cf = fine[64 * k + lane];
  const int pf = wave_incl_scan(cf);
  const int sf = abv + __builtin_amdgcn_readlane(pf, WAVE - 1) - pf + cf;
  const int f = __popcll(__ballot(sf >= need)) - 1;
  *bin = 64 * k + f;
  *above = __builtin_amdgcn_readlane(sf - cf, f);
  return tot;
}

// The 64 coarse sums of 4096 fine bins (coarse c: bins 64 c .. 64 c + 63), by the whole workgroup: thread t sums bins
// 8 t .. 8 t + 7, then its 8 lanes' sums add up by DPP (quad swaps and the half-row mirror). The fine bins are complete
// (a barrier before); a barrier after, before the coarse bins are read.
__device__ __forceinline__ void fu_coarse_sums(const int* fine, int* coarse) {
  const int t = threadIdx.x;
  const int4 a = reinterpret_cast<const int4*>(fine)[2 * t], b = reinterpret_cast<const int4*>(fine)[2 * t + 1];
  int v = a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w;
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  if ((t & 7) == 0) coarse[t >> 3] = v;
}
static_assert(FU_THREADS * 8 == 4096, "a thread's 8 fine bins");

// The same over 256 bins (lane l: bins 4 l .. 4 l + 3).
__device__ __forceinline__ int fu_wave_find256(const int* bins, int need, int* bin, int* above) {
  const int lane = threadIdx.x & (WAVE - 1);
  int v[4];
  *reinterpret_cast<int4*>(v) = *reinterpret_cast<const int4*>(bins + 4 * lane);
  const int m = v[0] + v[1] + v[2] + v[3];
  const int p = wave_incl_scan(m);
  const int tot = __builtin_amdgcn_readlane(p, WAVE - 1);
  const int sc = tot - p + m;
  if (need <= 0 || tot < need) {
    *bin = 0;
    *above = 0;
    return tot;
  }
  const int k = __popcll(__ballot(sc >= need)) - 1;
  int e = sc - m, bl = 4 * lane, al = 0;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    if (e < need && e + v[i] >= need) {
      bl = 4 * lane + i;
      al = e;
    }
    e += v[i];
  }
  *bin = __builtin_amdgcn_readlane(bl, k);
  *above = __builtin_amdgcn_readlane(al, k);
  return tot;
}

// Block-wide exclusive prefix (in thread order) of a packed per-thread count (two 16-bit fields; block totals below
// 65536), and the block total. scr: FU_WAVES ints. One barrier; the caller must pass one more before scr is written
// again.
__device__ __forceinline__ uint32_t fu_block_prefix(uint32_t mine, int* scr, uint32_t* total) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  const uint32_t incl = wave_incl_scan_u32(mine);
  if (lane == WAVE - 1) scr[wave] = (int)incl;
  __syncthreads();
  uint32_t before = incl - mine, tot = 0;
#pragma unroll
  for (int w = 0; w < FU_WAVES; ++w) {
    const uint32_t x = (uint32_t)scr[w];
    before += w < wave ? x : 0u;
    tot += x;
  }
  *total = tot;
  return before;
}

// Positions per workgroup in a row of L tokens: 32 ceil(L / 1024), at least one tile, at most 1024.
__device__ __forceinline__ int fu_kw(int L) {
  return min(FU_KEYS, max(FU_TILE, (L + FU_NW * FU_TILE - 1) / (FU_NW * FU_TILE) * FU_TILE));
}

// The workgroup's kw scores from LDS into the score output (positions kw j + e; none past the row's stride), for a
// row that selects from the key lists: written after barrier A, behind the selection's first loads, so that their
// write latency overlaps the selection instead of holding up the indexer's end (its bin search waits for the memory
// counter). The two-exchange form writes each tile's scores as it is scored, as those stores drain during the tiles.
__device__ __forceinline__ void fu_store_scores(const FusedArgs& a, const uint8_t* lds, int b, int j, int kw) {
  const float* sc = reinterpret_cast<const float*>(lds + L_SCS);
  float* srow = a.scores + (size_t)b * a.stride;
#pragma unroll
  for (int e = threadIdx.x; e < FU_KEYS; e += FU_THREADS)
    if (e < kw && j * kw + e < a.stride) srow[j * kw + e] = sc[e];
}

// Whether a row of L tokens takes the one-exchange selection from the key lists (workgroup-uniform): every list holds
// all its workgroup's keys (kw <= LCAP: the pooled form always), or the workgroups select at most 80 keys each on
// average.
template <bool POOL = false>
__device__ __forceinline__ bool fu_lists_on(const FusedArgs& a, int L) {
  const int kw = fu_kw(L);
  return POOL || kw <= FU_LCAP || (long)a.keep * kw * 8 <= 5L * FU_LM * L;
}

// This thread's two keys (positions tid, tid + 512 of the workgroup's block; 0: not selectable, as every position past
// the block's kw is).
__device__ __forceinline__ void fu_my_keys(const uint8_t* lds, uint32_t (&key)[2]) {
  const float* sc = reinterpret_cast<const float*>(lds + L_SCS);
  const float v0 = sc[threadIdx.x], v1 = sc[threadIdx.x + FU_THREADS];
  key[0] = order_key(v0) & (0u - (uint32_t)(v0 > VISIBLE));
  key[1] = order_key(v1) & (0u - (uint32_t)(v1 > VISIBLE));
}

// Stage 1: the indexer scores of positions kw j .. kw j + kw - 1 of row b (L: the row's length, kw = fu_kw(L)): the
// block's tiles (32 keys each) go to the waves in turn, wave v taking tiles v, v + 8, v + 16, v + 24 of the block (the
// ones the block has) and streaming them FU_AHEAD ahead of its MFMAs. LDS holds the scores of all 1024 positions of
// the workgroup's range, NEG_INF past the block. The pooled form (POOL) scores pools: a position is a pool, its key
// 128 bf16 with no scale at page row p >> ppp_shift (trnrt/models/mla.py:615-630), the arithmetic of the bf16 decode
// indexer; its key list holds every key of the block, so it writes no bin list (no two-exchange selection reads one).
// The pooled step's pool-key write (WRITE; trnrt/models/mla.py:1262-1296 `write_pool_keys` with
// trnrt/models/glm5_next.py:151-160 `pool_keys`, the arithmetic of pool_keys_kernel): the row's written token's pool
// key, pk[d] = bf16( sum_t bf16( bf16(softmax_t(g_t[d] + ape[t, d])) * k_t[d] ) ) over its kpool cached indexer rows
// [key 128 | gate logits 128], from one wave (2 channels a lane), stored as kpool pieces of 128 / kpool values, piece
// i into the slot of the pool's i-th token (a padded row, slot in the null page: every piece into its own slot);
// returns this lane's two channels as bf16 bits (the key's 128 values across the wave). Loads first (fu_pool_key_load),
// so that they overlap the wave's key tiles.
constexpr int PKF_MAXKP = 8;
struct PoolKeyRows {
  float k[PKF_MAXKP][2], g[PKF_MAXKP][2], ape[PKF_MAXKP][2];
  long first;  // the slot of the pool's token 0 (a padded row: its own slot)
  bool real;
};
template <int KP>
__device__ __forceinline__ long fu_pool_slot(const FusedArgs& a, const PoolKeyRows& r, int t) {
  const long sl = r.real ? r.first + min(t, KP - 1) : r.first;
  return min(max(sl, 0L), (long)a.num_slots - 1);  // in range whatever the inputs
}
template <int KP>
__device__ __forceinline__ void fu_pool_key_load_t(const FusedArgs& a, int pos, long own, PoolKeyRows& r) {
  constexpr int Di = FU_D;
  const int lane = threadIdx.x & (WAVE - 1);
  r.real = own >= a.page_size;
  r.first = r.real ? own - (pos & (KP - 1)) : own;
#pragma unroll
  for (int t = 0; t < KP; ++t) {
    const long slot = fu_pool_slot<KP>(a, r, t);
    const size_t base = (size_t)slot * a.pk_width;
    if (a.pk_fp8) {
      const uint8_t* row = static_cast<const uint8_t*>(a.pk_rows) + base;
      const float sc = a.pk_scale ? a.pk_scale[slot] : 1.0f;
      const auto kf = __builtin_amdgcn_cvt_pk_f32_fp8(*reinterpret_cast<const uint16_t*>(row + 2 * lane), false);
      const auto gf = __builtin_amdgcn_cvt_pk_f32_fp8(*reinterpret_cast<const uint16_t*>(row + Di + 2 * lane), false);
      // the reference reads the e4m3 rows in bf16 (exact); a per-token scale is applied in fp32, rounded to bf16
      r.k[t][0] = __uint_as_float((uint32_t)f32_to_bf16_bits(kf[0] * sc) << 16);
      r.k[t][1] = __uint_as_float((uint32_t)f32_to_bf16_bits(kf[1] * sc) << 16);
      r.g[t][0] = __uint_as_float((uint32_t)f32_to_bf16_bits(gf[0] * sc) << 16);
      r.g[t][1] = __uint_as_float((uint32_t)f32_to_bf16_bits(gf[1] * sc) << 16);
    } else {
      const uint16_t* row = static_cast<const uint16_t*>(a.pk_rows) + base;
      const uint32_t kw = *reinterpret_cast<const uint32_t*>(row + 2 * lane);
      const uint32_t gw = *reinterpret_cast<const uint32_t*>(row + Di + 2 * lane);
      r.k[t][0] = __uint_as_float(kw << 16), r.k[t][1] = __uint_as_float(kw & 0xffff0000u);
      r.g[t][0] = __uint_as_float(gw << 16), r.g[t][1] = __uint_as_float(gw & 0xffff0000u);
    }
    r.ape[t][0] = a.pk_ape[t * Di + 2 * lane];
    r.ape[t][1] = a.pk_ape[t * Di + 2 * lane + 1];
  }
}
template <int KP>
__device__ __forceinline__ uint32_t fu_pool_key_write_t(const FusedArgs& a, const PoolKeyRows& r) {
  constexpr int Di = FU_D;
  const int lane = threadIdx.x & (WAVE - 1);
  uint32_t out = 0;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float x[KP], m = -INFINITY;
#pragma unroll
    for (int t = 0; t < KP; ++t) {
      x[t] = r.g[t][c] + r.ape[t][c];
      m = fmaxf(m, x[t]);
    }
    float e[KP], sum = 0.0f;
#pragma unroll
    for (int t = 0; t < KP; ++t) {
      e[t] = expf(x[t] - m);
      sum += e[t];
    }
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < KP; ++t) {
      const float wt = __uint_as_float((uint32_t)f32_to_bf16_bits(e[t] / sum) << 16);
      acc += __uint_as_float((uint32_t)f32_to_bf16_bits(wt * r.k[t][c]) << 16);
    }
    out |= (uint32_t)f32_to_bf16_bits(acc) << (16 * c);
  }
  // piece i (channels i Di / kp ..) into slot i: this lane's two channels
  constexpr int per = Di / KP;
  const int piece = (2 * lane) / per;
  uint16_t* pk = reinterpret_cast<uint16_t*>(const_cast<uint8_t*>(a.k));
  *reinterpret_cast<uint32_t*>(pk + (size_t)fu_pool_slot<KP>(a, r, piece) * per + (2 * lane - piece * per)) = out;
  return out;
}
constexpr int FU_STEP_KP = 4;  // the kpool the one-launch step takes (GLM's); others write with the write's kernel
constexpr int L_PKEY = 4096;  // stage 1 of the pooled step: the written pool's key [128] bf16

template <int MT, bool POOL = false, bool WRITE = false>
__device__ __forceinline__ void fu_indexer(const FusedArgs& a, uint8_t* lds, int b, int j, int L) {
  static_assert(!WRITE || POOL, "the pool-key write belongs to the pooled form");
  using FF = FuForm<POOL>;
  uint16_t* qs = reinterpret_cast<uint16_t*>(lds + L_QS);
  float* wsh = reinterpret_cast<float*>(lds + L_WS);
  int* hs = reinterpret_cast<int*>(lds + L_HS);
  int* hsc = reinterpret_cast<int*>(lds + L_HSC);
  float* scs = reinterpret_cast<float*>(lds + L_SCS);
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int jk = lane & 31, h = lane >> 5;
  const int Hi = a.Hi;
  float* srow = a.scores + (size_t)b * a.stride;
  // a row that selects from the key lists writes its scores after barrier A; the others as each tile is scored
  const bool lists = fu_lists_on<POOL>(a, L);
  uint32_t* plst = a.lst + ((size_t)b * FU_NW + j) * FF::LROW;  // the pooled form's key list

  // the pooled step: the row's written position and its slot, loaded with the queries
  int pk_pos = 0;
  long pk_own = 0;
  if (WRITE) {
    pk_pos = a.positions[b];
    pk_own = a.slot_mapping[b];
  }
  // the queries' loads (32 MT heads of 16 pieces: MT per thread), the weights, the tiles' pages
  u32x4 qv[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    const int i = tid + FU_THREADS * r;
    const int head = i >> 4, c = i & 15;
    qv[r] = *reinterpret_cast<const u32x4*>(a.q_idx + ((size_t)b * Hi + min(head, Hi - 1)) * FU_D + 8 * c);
  }
  const float wv = a.w[(size_t)b * Hi + min(tid, Hi - 1)];
  const int kw = fu_kw(L), nt = kw / FU_TILE;  // the block's positions and tiles
  // tile i of this wave: the block's tile wave + 8 i, the row's tile t_begin + 8 i; it holds keys of the row when
  // wave + 8 i < nt and its first position is below L
  const int t_begin = j * nt + wave;
  const bool live = wave < nt && t_begin * FU_TILE < L;  // wave-uniform: any of its keys in the row
  auto in_row = [&](int i) __attribute__((always_inline)) {
    return wave + FU_WAVES * i < nt && (t_begin + FU_WAVES * i) * FU_TILE < L;
  };
  const int* trow = a.table + (size_t)b * a.max_pages;
  int pages = 0;
  if (POOL) {
    // a tile of 32 pools spans two page rows of 16 pools (or lies inside one of 32 or more): lane 2 i + u holds the
    // page of tile i's pools 32 t + 16 u ..
    const int i = min(lane >> 1, FU_TPW - 1), u = lane & 1;
    const int t = t_begin + FU_WAVES * i;
    const int pg = trow[min((t * FU_TILE + 16 * u) >> a.ppp_shift, a.max_pages - 1)];
    pages = in_row(i) ? safe_page(pg, a.num_pages) : 0;
  } else {
    const int i = min(lane, FU_TPW - 1);
    const int t = t_begin + FU_WAVES * i;
    const int pg = trow[min((t * FU_TILE) >> a.page_shift, a.max_pages - 1)];
    pages = in_row(i) ? safe_page(pg, a.num_pages) : 0;
  }
  // the pooled step: the written token's pool kP, its key written by the wave whose tile holds kP (the last block's
  // last wave when kP is past the row's blocks) and scored from the new key when the pool is complete (kP < L)
  int kP = 0;
  bool kwave = false;
  PoolKeyRows pkr;
  if (WRITE) {
    kP = max(pk_pos, 0) >> a.kp_shift;
    const int jw = min(kP / kw, FU_NW - 1), tw = min(max(kP - jw * kw, 0) / FU_TILE, FU_WAVES - 1);
    kwave = j == jw && wave == tw;  // wave-uniform
  }
  u32x4 kv[FU_TPW][FF::KV];
  float ksc[FU_TPW];
  auto tile_loads = [&](int i) __attribute__((always_inline)) {
    const int t0 = (t_begin + FU_WAVES * i) * FU_TILE;
    if (POOL) {
      const int pa = __builtin_amdgcn_readlane(pages, 2 * i), pb = __builtin_amdgcn_readlane(pages, 2 * i + 1);
      const int ppp = 1 << a.ppp_shift;
      const size_t row = (size_t)(in_row(i) ? (jk < 16 ? pa : pb) : 0) * ppp + ((t0 + jk) & (ppp - 1));
      const uint8_t* kp = a.k + row * (2 * FU_D) + 128 * h;
#pragma unroll
      for (int c = 0; c < FF::KV; ++c) kv[i][c] = *reinterpret_cast<const u32x4*>(kp + 16 * c);
      ksc[i] = 1.0f;
    } else {
      const int page = __builtin_amdgcn_readlane(pages, i);
      const size_t slot = in_row(i) ? (size_t)page * a.page_size + (t0 & (a.page_size - 1)) + jk : (size_t)jk;
      const uint8_t* kp = a.k + slot * FU_D + 64 * h;
#pragma unroll
      for (int c = 0; c < FF::KV; ++c) kv[i][c] = *reinterpret_cast<const u32x4*>(kp + 16 * c);
      ksc[i] = a.ks[slot];
    }
  };
  if (live) {
#pragma unroll
    for (int i = 0; i < FU_AHEAD; ++i) tile_loads(i);
  }
  if (WRITE && kwave) fu_pool_key_load_t<FU_STEP_KP>(a, pk_pos, pk_own, pkr);  // the written pool's rows, behind the key tiles

#pragma unroll
  for (int r = 0; r < MT; ++r) {
    const int i = tid + FU_THREADS * r;
    const int head = i >> 4, c = i & 15;
    *reinterpret_cast<u32x4*>(&qs[head * FU_QROW + 8 * c]) = head < Hi ? qv[r] : u32x4{0u, 0u, 0u, 0u};
  }
  if (tid < 32 * MT) wsh[tid] = tid < Hi ? wv : 0.0f;
  for (int i = tid; i < FU_HBINS; i += FU_THREADS) hs[i] = 0;
  if (tid < 64) hsc[tid] = 0;
  int* scr = reinterpret_cast<int*>(lds + L_MISC);
  __syncthreads();
  if (WRITE && kwave) {
    const uint32_t key2 = fu_pool_key_write_t<FU_STEP_KP>(a, pkr);
    if (kP < L) reinterpret_cast<uint32_t*>(lds + L_PKEY)[lane] = key2;
  }

  if (live) {
    bf16x8 qa[MT][8];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int s = 0; s < 8; ++s)
        qa[m][s] = as_bf16x8(*reinterpret_cast<const uint4*>(&qs[(32 * m + jk) * FU_QROW + 64 * h + 8 * s]));
    float wr[MT][16];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) wr[m][r] = wsh[32 * m + 8 * (r >> 2) + 4 * h + (r & 3)];
#pragma unroll
    for (int i = 0; i < FU_TPW; ++i) {
      if (i + FU_AHEAD < FU_TPW) {
        // tile i has arrived (the later tiles in flight may still be outstanding): issue tile i + FU_AHEAD (the
        // compiler's own wait before tile i's first use keeps the data exact)
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(FF::TILE_LOADS * (FU_AHEAD - 1)));
        __builtin_amdgcn_sched_barrier(0);
        tile_loads(i + FU_AHEAD);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (WRITE && i == 0 && kwave && kP < L) {
        // the written pool's two lanes take its new key (the tile's loads read the cache before the write)
        if (jk == (kP & (FU_TILE - 1))) {
          const u32x4* nk = reinterpret_cast<const u32x4*>(lds + L_PKEY + 128 * h);
#pragma unroll
          for (int c = 0; c < FF::KV; ++c) kv[0][c] = nk[c];
        }
      }
      const int pos = (t_begin + FU_WAVES * i) * FU_TILE + jk, e = (wave + FU_WAVES * i) * FU_TILE + jk;
      const bool mine = wave + FU_WAVES * i < nt;  // a position of this workgroup's block
      f32x16 acc[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        bf16x8 kb;
        if (POOL) {
          kb = __builtin_bit_cast(bf16x8, kv[i][s]);
        } else {
          const u32x4 k4 = kv[i][s >> 1];
          kb = (s & 1) ? fp8x8_to_bf16x8(k4[2], k4[3]) : fp8x8_to_bf16x8(k4[0], k4[1]);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[m][s], kb, acc[m], 0, 0, 0);
      }
      float part = 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) part = fmaf(wr[m][r], relu(acc[m][r]), part);
      part += __shfl_xor(part, 32, WAVE);
      const float v = mine && pos < L ? (POOL ? part : part * ksc[i]) : NEG_INF;
      if (h == 0) {
        if (!lists && mine && pos < a.stride) srow[pos] = v;
        scs[e] = v;
        if (POOL && mine) plst[e] = order_key(v) & (0u - (uint32_t)(v > VISIBLE));
        if (v > VISIBLE) atomicAdd(&hs[order_key(v) >> 20], 1);
      }
    }
  } else {
    // every key of this wave is past the row or the block: NEG_INF
    for (int x = lane; x < FU_TPW * FU_TILE; x += WAVE) {
      const int lt = wave + FU_WAVES * (x / FU_TILE);  // the tile of the block
      const int pos = (j * nt + lt) * FU_TILE + (x & (FU_TILE - 1));
      if (!lists && lt < nt && pos < a.stride) srow[pos] = NEG_INF;
      if (POOL && lt < nt) plst[lt * FU_TILE + (x & (FU_TILE - 1))] = 0u;
      scs[lt * FU_TILE + (x & (FU_TILE - 1))] = NEG_INF;
    }
  }
  // positions past the 32 blocks (32 kw) of a wider score row are never keys of the row
  for (int p = FU_NW * kw + j * FU_THREADS + tid; p < a.stride; p += FU_NW * FU_THREADS) srow[p] = NEG_INF;
  if (POOL) {
    // the block's highest nonzero histogram bins after its keys (thread t: bins 8 t .. 8 t + 7; its place among the
    // nonzero bins from the top, from a block prefix of the counts)
    __syncthreads();
    int hv[8];
    *reinterpret_cast<int4*>(hv) = *reinterpret_cast<const int4*>(hs + 8 * tid);
    *reinterpret_cast<int4*>(hv + 4) = *reinterpret_cast<const int4*>(hs + 8 * tid + 4);
    uint32_t nz = 0, tot;
#pragma unroll
    for (int i = 0; i < 8; ++i) nz += hv[i] != 0;
    uint32_t o = fu_block_prefix(nz, scr, &tot);
    uint32_t* pb = plst + FF::LCAP;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (hv[i]) {
        const int d = (int)tot - 1 - (int)o;
        if (d < FU_PBINS) pb[d] = ((uint32_t)(8 * tid + i) << 16) | (uint32_t)hv[i];
        ++o;
      }
    if (tid >= (int)tot && tid < FU_PBINS) pb[tid] = 0u;
    return;
  }
  __syncthreads();
  // the histogram's nonzero bins into the workgroup's bin list (thread t: bins 8 t .. 8 t + 7), in bin order, and
  // the workgroup's key list: the bin of its FU_LM-th largest key, then its keys from that bin up (or from the next
  // bin up when that would overflow the list; every key when they fit), the first half's by thread, then the second
  // half's
  int hv[8];
  *reinterpret_cast<int4*>(hv) = *reinterpret_cast<const int4*>(hs + 8 * tid);
  *reinterpret_cast<int4*>(hv + 4) = *reinterpret_cast<const int4*>(hs + 8 * tid + 4);
  int lbin = FU_HBINS, lcnt = 0;  // no list
  if (POOL) {
    lbin = 0;  // every key of the block (at most 256), whatever their bins; counted by the prefix below
  } else if (lists) {
    // the key list's bin search over the histogram and its coarse sums (summed here: a row's keys fall in few
    // coarse bins, and adding each key to its coarse bin queued the tiles' atomics on a few words)
    {
      int v = hv[0] + hv[1] + hv[2] + hv[3] + hv[4] + hv[5] + hv[6] + hv[7];
      v += dpp<0xb1>(v);
      v += dpp<0x4e>(v);
      v += dpp<0x141>(v);
      if ((tid & 7) == 0) hsc[tid >> 3] = v;
    }
    __syncthreads();
    int lb, labove;
    const int nv = fu_wave_find(hs, hsc, FU_LM, &lb, &labove);
    lbin = 0;
    lcnt = nv;
    if (nv > FU_LCAP) {
      const int nb = labove + hs[lb];
      lbin = nb <= FU_LCAP ? lb : lb + 1;
      lcnt = nb <= FU_LCAP ? nb : labove;
    }
  }
  uint32_t key[2] = {0u, 0u};
  if (lists) fu_my_keys(lds, key);
  const bool in0 = key[0] != 0u && (int)(key[0] >> 20) >= lbin, in1 = key[1] != 0u && (int)(key[1] >> 20) >= lbin;
  uint32_t nz = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) nz += hv[i] != 0;
  // (nonzero bins) << 20 | (listed keys of the first half) << 10 | (of the second half): at most 1024, 512, 512
  uint32_t tot;
  const uint32_t before = fu_block_prefix((nz << 20) | ((uint32_t)in0 << 10) | (uint32_t)in1, scr, &tot);
  uint32_t* hl = a.hl + ((size_t)b * FU_NW + j) * FU_HROW;
  uint32_t* lrow = a.lst + ((size_t)b * FU_NW + j) * FF::LROW;
  const int nzt = (int)(tot >> 20);
  if (POOL) lcnt = (int)(((tot >> 10) & 1023u) + (tot & 1023u));
  uint32_t o = before >> 20;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (hv[i]) {
      const uint32_t e = ((uint32_t)(8 * tid + i) << 16) | (uint32_t)hv[i];
      if (!POOL) hl[1 + o] = e;
      const int d = nzt - 1 - (int)o;  // this bin's place among the nonzero bins from the top
      if (lists && d < FU_LBINS) lrow[4 + d] = e;
      ++o;
    }
  if (lists) {
    if (in0)
      *reinterpret_cast<uint2*>(lrow + FU_LHDR + 2 * ((before >> 10) & 1023u)) = uint2{key[0], (uint32_t)tid};
    if (in1)
      *reinterpret_cast<uint2*>(lrow + FU_LHDR + 2 * (((tot >> 10) & 1023u) + (before & 1023u))) =
          uint2{key[1], (uint32_t)(tid + FU_THREADS)};
    if (tid >= nzt && tid < FU_LBINS) lrow[4 + tid] = 0u;
    if (tid == 0) *reinterpret_cast<uint4*>(lrow) = uint4{(uint32_t)lcnt, (uint32_t)lbin, 0u, 0u};
  }
  if (!POOL && tid == 0) hl[0] = (uint32_t)nzt;
}

// Stage 2: the first level from the row histogram, this workgroup's keys above it counted and its candidates written.
__device__ __forceinline__ void fu_classify(const FusedArgs& a, uint8_t* lds, int b, int j) {
  FuState& st = *reinterpret_cast<FuState*>(lds + L_STATE);
  int* scr = reinterpret_cast<int*>(lds + L_MISC);
  const int tid = threadIdx.x;
  constexpr int PER = FU_HBINS / FU_THREADS;  // 8 bins per thread
  const int wave = tid / WAVE, lane = tid & (WAVE - 1);
  // the row histogram in LDS from every workgroup's bin list (the first 256 words of each straight into LDS; load
  // i: list i, lane l words 4 l .. 4 l + 3)
  uint32_t* hls = reinterpret_cast<uint32_t*>(lds + L_HLS);
  int* rh = reinterpret_cast<int*>(lds + L_HS);
  const uint32_t* hlg = a.hl + (size_t)b * FU_NW * FU_HROW;
  for (int i = wave; i < FU_NW; i += FU_WAVES)
    __builtin_amdgcn_global_load_lds(hlg + (size_t)i * FU_HROW + 4 * lane,
                                     (__attribute__((address_space(3))) void*)(hls + FU_HSTAGE * i), 16, 0,
                                     FU_AUX_PLAIN);
  *reinterpret_cast<int4*>(rh + PER * tid) = int4{0, 0, 0, 0};
  *reinterpret_cast<int4*>(rh + PER * tid + 4) = int4{0, 0, 0, 0};
  uint32_t key[2];
  fu_my_keys(lds, key);
  if (tid == 0) scr[8] = -1;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  {
    const int w = tid >> 4, q = tid & 15;  // list w's entries q, q + 16, ...
    const uint32_t* lw = hls + FU_HSTAGE * w;
    const int n = min((int)lw[0], FU_KEYS);  // (bounded: a list read after a wait that gave up may be stale)
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = lw[1 + q + 16 * i];  // within the staged 256 words
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (q + 16 * i < n) atomicAdd(&rh[(v[i] >> 16) & (FU_HBINS - 1)], (int)(v[i] & 0xFFFFu));
    for (int e = q + 128; e < n; e += 16) {
      const uint32_t x = e + 1 < FU_HSTAGE ? lw[1 + e] : hlg[(size_t)w * FU_HROW + 1 + e];
      atomicAdd(&rh[(x >> 16) & (FU_HBINS - 1)], (int)(x & 0xFFFFu));
    }
  }
  __syncthreads();
  int hb[PER];
  *reinterpret_cast<int4*>(hb) = *reinterpret_cast<const int4*>(rh + PER * tid);
  *reinterpret_cast<int4*>(hb + 4) = *reinterpret_cast<const int4*>(rh + PER * tid + 4);
  int c0, above0;
  const int nvis = fu_find_bin<PER>(hb, a.keep, scr, &c0, &above0);
  if (nvis <= a.keep) c0 = -1;  // every selectable key is selected
  bool sure[2], cand[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int bin = (int)(key[e] >> 20);
    sure[e] = key[e] != 0u && bin > c0;
    cand[e] = key[e] != 0u && bin == c0;
  }
  // the bitmap of the positions above c0: wave v's ballots cover positions 64 v .. + 63 and 512 + 64 v .. + 63
  uint32_t* blk = a.cand + ((size_t)b * FU_NW + j) * FU_CROW;
  const uint64_t bm0 = __ballot(sure[0]), bm1 = __ballot(sure[1]);
  if (lane == 0) {
    *reinterpret_cast<uint64_t*>(blk + 1 + 2 * wave) = bm0;
    *reinterpret_cast<uint64_t*>(blk + 1 + FU_BMW / 2 + 2 * wave) = bm1;
  }
  __syncthreads();  // every thread has read scr (the bin search) before it is rewritten
  // (keys above c0) << 20 | (candidates in the first half) << 10 | (candidates in the second half): the candidates
  // in position order are the first half's by thread, then the second half's
  uint32_t tot;
  const uint32_t before = fu_block_prefix(((uint32_t)(sure[0] + sure[1]) << 20) | ((uint32_t)cand[0] << 10) |
                                              (uint32_t)cand[1],
                                          scr, &tot);
  const int n0 = (int)((tot >> 10) & 1023u), n1 = (int)(tot & 1023u);
  uint32_t* crow = blk + 1 + FU_BMW;
  if (cand[0]) crow[(before >> 10) & 1023u] = ((key[0] & 0xFFFFFu) << 10) | (uint32_t)tid;
  if (cand[1]) crow[n0 + (int)(before & 1023u)] = ((key[1] & 0xFFFFFu) << 10) | (uint32_t)(tid + FU_THREADS);
  if (tid == 0) {
    blk[0] = ((tot >> 20) << 16) | (uint32_t)(n0 + n1);
    st.c0 = c0;
    st.above0 = above0;
    st.nvis = nvis;
  }
}

// The end of the selection, shared by its two forms: every workgroup's selected positions are in the bitmaps at L_SB
// (bit e of workgroup w's: position kw w + e; lane w of every wave: workgroup w's selected count selw and first output
// index offw), the pages of the positions from page pg0 on at L_SPG (this wave's loads of them may be in flight). The
// workgroup writes the indices of its split's outputs [o0, o1), lists their cache slots at FuAtt<HPW>::L_P, stages the
// attention's queries and returns the split's selected count.
template <int HPW>
__device__ __forceinline__ int fu_split_slots(const FusedArgs& a, uint8_t* lds, int b, int j, int kw, int selw,
                                              int offw, int o0, int o1, int cnt_row, int pg0,
                                              const u32x4 (&qv)[FuAtt<HPW>::QPT], float* live_bias) {
  using AT = FuAtt<HPW>;
  constexpr int QPT = AT::QPT;
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(lds + L_SB);
  int* pb = reinterpret_cast<int*>(lds + L_PB);
  const int* spg = reinterpret_cast<const int*>(lds + L_SPG);
  int* slot_l = reinterpret_cast<int*>(lds + AT::L_P);
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 4, q = tid & 15;
  const int hg = j % a.HG, s = j / a.HG;
  const bool active = s < a.S;
  // exclusive prefix popcounts of each block's selected bitmap (thread (w, q): words 2 q, 2 q + 1)
  {
    const int c_a = __builtin_popcount(sb[FU_BMW * w + 2 * q]), c_b = __builtin_popcount(sb[FU_BMW * w + 2 * q + 1]);
    const int incl = row_incl_scan(c_a + c_b);
    pb[FU_BMW * w + 2 * q] = incl - c_a - c_b;
    pb[FU_BMW * w + 2 * q + 1] = incl - c_b;
  }
  // the queries into LDS for stage 4, head pc / 72, elements 8 (pc % 72) .. of piece pc (before the index stores
  // below: a wait for the queries' loads there would also wait for those stores)
  if (active) {
    uint16_t* qs = reinterpret_cast<uint16_t*>(lds + AT::L_QST);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int pc = tid + FU_THREADS * i;
      if (pc < HPW * FU_DQK / 8)
        *reinterpret_cast<u32x4*>(qs + (pc / (FU_DQK / 8)) * FU_AQROW + 8 * (pc % (FU_DQK / 8))) = qv[i];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's page loads have landed
  __syncthreads();
  // the split's sources exactly: the workgroups whose outputs meet [o0, o1); each thread takes a byte of their
  // bitmaps (at most 8 selected positions, so a dense selection costs no more than a sparse one) and lists each
  // selected position whose output falls in the split
  int* irow = a.idx + (size_t)b * a.keep;
  const uint64_t ms = __ballot(lane < FU_NW && selw > 0 && offw < o1 && offw + selw > o0);
  if (ms) {
    const int wa = (int)__builtin_ctzll(ms), nbytes = 4 * FU_BMW * (64 - (int)__builtin_clzll(ms) - wa);
    for (int k = tid; k < nbytes; k += FU_THREADS) {
      const int sw = wa + k / (4 * FU_BMW), i = (k / 4) % FU_BMW, by = 8 * (k & 3);
      const uint32_t word = sb[FU_BMW * sw + i];
      uint32_t bits = (word >> by) & 255u;
      int o = __shfl(offw, sw, WAVE) + pb[FU_BMW * sw + i] + __builtin_popcount(word & ((1u << by) - 1u));
      // the word's 32 positions lie in one page (kw a multiple of 32, pages of at least 32 tokens)
      const int p0 = kw * sw + 32 * i;
      const int sbase =
          safe_page(spg[(p0 >> a.page_shift) - pg0], a.num_pages) * a.page_size + (p0 & (a.page_size - 1)) + by;
      while (bits) {
        const int bit = __builtin_ctz(bits);
        bits &= bits - 1u;
        if (o >= o0 && o < o1) {
          slot_l[o - o0] = sbase + bit;
          if (hg == 0) irow[o] = p0 + by + bit;
        }
        ++o;
      }
    }
  }
  // the outputs past the count, and the count
  if (hg == 0)
    for (int o = max(o0, cnt_row) + tid; o < o1; o += FU_THREADS) irow[o] = 0;
  if (j == 0 && tid == 0) a.cnt[b] = cnt_row;
  // the split's live slots; a row with none attends position 0 masked (its lse is NEG_INF)
  int n_slots = max(min(o1, cnt_row) - o0, 0);
  *live_bias = 0.0f;
  if (active && cnt_row == 0 && s == 0) {
    n_slots = 1;
    *live_bias = NEG_INF;
    if (tid == 0) slot_l[0] = safe_page(a.table[(size_t)b * a.max_pages], a.num_pages) * a.page_size;
  }
  __syncthreads();  // the slot list
  return n_slots;
}

// Stage 3: the exact selection and this workgroup's split of it. Every workgroup reads the first 128 words of every
// candidate block (the counts, the bitmap of the positions above c0, the first 95 candidates) and finds T (the
// keep-th largest key), the ties at T to take and each workgroup's output offset; the candidates taken join the
// bitmaps, whose prefix popcounts give every selected position its output index, so the workgroup lists the slots of
// its split's outputs [o0, o1) itself (and writes their indices): no further hand-off between workgroups. Returns the
// split's selected count; its cache slots are in LDS at FuAtt<HPW>::L_P.
template <int HPW>
__device__ __forceinline__ int fu_select(const FusedArgs& a, uint8_t* lds, int b, int j, int L,
                                         u32x4 (&qv)[FuAtt<HPW>::QPT], float* live_bias) {
  using AT = FuAtt<HPW>;
  constexpr int QPT = AT::QPT;
  FuState& st = *reinterpret_cast<FuState*>(lds + L_STATE);
  int* scr = reinterpret_cast<int*>(lds + L_MISC);
  int* bins = reinterpret_cast<int*>(lds + L_BINS);
  int* bins2 = reinterpret_cast<int*>(lds + L_BINS2);
  int* spg = reinterpret_cast<int*>(lds + L_SPG);
  const uint32_t* cb = reinterpret_cast<const uint32_t*>(lds + L_CB);
  uint32_t* sb = reinterpret_cast<uint32_t*>(lds + L_SB);
  int* slot_l = reinterpret_cast<int*>(lds + AT::L_P);
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int c0 = st.c0;
  const int hg = j % a.HG, s = j / a.HG;
  const bool active = s < a.S;  // workgroup-uniform: a workgroup past the last split only helps with the barriers
  const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
  const int kw = fu_kw(L);
  const uint32_t* cblk = a.cand + (size_t)b * FU_NW * FU_CROW;
  // the staged words of every block straight into LDS (load i: blocks 2 i, 2 i + 1; lane l words 4 (l % 32) .. + 3
  // of block 2 i + l / 32)
  for (int i = wave; i < FU_NW / 2; i += FU_WAVES)
    __builtin_amdgcn_global_load_lds(cblk + (size_t)(2 * i + (lane >> 5)) * FU_CROW + 4 * (lane & 31),
                                     (__attribute__((address_space(3))) void*)(cb + 2 * FU_CSTAGE * i), 16, 0,
                                     FU_AUX_PLAIN);
  // the attention's HPW heads' queries: their QPT loads go out after the block loads (kept in that order) and are
  // used after the selection
  __builtin_amdgcn_sched_barrier(0);
  if (active) {
    const u32x4* qsrc = reinterpret_cast<const u32x4*>(a.q + ((size_t)b * a.H + HPW * hg) * FU_DQK);
#pragma unroll
    for (int i = 0; i < QPT; ++i) qv[i] = qsrc[min(tid + FU_THREADS * i, HPW * FU_DQK / 8 - 1)];
  }
  for (int i = tid; i < 4096; i += FU_THREADS) bins[i] = 0;
  if (tid < 256) bins2[tid] = 0;
  if (tid < AT::SPLIT) slot_l[tid] = 0;  // padding rows read slot 0
  if (tid == 0) scr[8] = -1;
  __builtin_amdgcn_sched_barrier(0);
  if (active)
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(QPT));  // the block loads (the queries may still be out)
  else
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
  __syncthreads();
  // thread (w, q) = (tid / 16, tid % 16): block w's bitmap words 2 q, 2 q + 1 and its candidates q, q + 16, ...
  const int w = tid >> 4, q = tid & 15;
  const uint32_t* cw = cb + FU_CSTAGE * w;
  const int nc = min((int)(cw[0] & 0xFFFFu), FU_KEYS);  // (bounded, as the bin lists above)
  sb[FU_BMW * w + 2 * q] = cw[1 + 2 * q];
  sb[FU_BMW * w + 2 * q + 1] = cw[2 + 2 * q];
  auto cand_at = [&](int e) __attribute__((always_inline)) {
    return e < FU_CSTAGED ? cw[1 + FU_BMW + e] : cblk[(size_t)w * FU_CROW + 1 + FU_BMW + e];
  };
  const uint32_t cq = q < nc ? cw[1 + FU_BMW + q] : 0u;  // this thread's first candidate (most blocks have <= 16)
  // lane w of every wave: block w's counts; the sources the split can draw on whatever T turns out to be (block w's
  // outputs lie in [sum of na before it, sum of na + nc up to it)), whose pages load while T is found
  const int ww = lane & (FU_NW - 1);
  const uint32_t cnw = cb[FU_CSTAGE * ww];
  const int nav = lane < FU_NW ? (int)(cnw >> 16) : 0, ncv = lane < FU_NW ? (int)(cnw & 0xFFFFu) : 0;
  const int lo = wave_incl_scan(nav) - nav, hi = wave_incl_scan(nav + ncv);
  const uint64_t mc = __ballot(lane < FU_NW && lo < o1 && hi > o0 && kw * lane < L);
  const int wa0 = mc ? (int)__builtin_ctzll(mc) : 0, nsrc0 = mc ? 64 - (int)__builtin_clzll(mc) - wa0 : 0;
  const int pg0 = (kw * wa0) >> a.page_shift;
  {
    // the pages from the first source block's first position to the last one's end (at most 1024: pages of at
    // least 32 tokens over at most 32,768 positions)
    const int npg = nsrc0 ? ((kw * (wa0 + nsrc0) + a.page_size - 1) >> a.page_shift) - pg0 : 0;
    const int* trow = a.table + (size_t)b * a.max_pages;
    for (int c = wave; WAVE * c < npg; c += FU_WAVES) {
      const int i = WAVE * c + lane;
      if (i < npg)
        __builtin_amdgcn_global_load_lds(trow + min(pg0 + i, a.max_pages - 1),
                                         (__attribute__((address_space(3))) void*)(spg + WAVE * c), 4, 0, 0);
    }
  }
  uint32_t T = 0u;
  int room = 0;
  int gt = 0, eq = 0;
  if (c0 >= 0) {
    // the candidates' low 20 key bits: 12 then 8
    if (q < nc) atomicAdd(&bins[(cq >> 18) & 4095], 1);
    for (int e = q + 16; e < nc; e += 16) atomicAdd(&bins[(cand_at(e) >> 18) & 4095], 1);
    __syncthreads();
    constexpr int P1 = 4096 / FU_THREADS;
    int hb[P1];
    *reinterpret_cast<int4*>(hb) = *reinterpret_cast<const int4*>(bins + P1 * tid);
    *reinterpret_cast<int4*>(hb + 4) = *reinterpret_cast<const int4*>(bins + P1 * tid + 4);
    int c1, above1;
    int need = a.keep - st.above0;
    fu_find_bin<P1>(hb, need, scr, &c1, &above1);
    need -= above1;
    uint32_t tlow;
    if (need >= bins[c1]) {
      // every key of bin c1 is taken: T is the bin's lowest key, and all its ties
      tlow = (uint32_t)c1 << 8;
      room = need;
    } else {
      __syncthreads();
      if (tid == 0) scr[8] = -1;
      if (q < nc && ((cq >> 18) & 4095) == (uint32_t)c1) atomicAdd(&bins2[(cq >> 10) & 255], 1);
      for (int e = q + 16; e < nc; e += 16) {
        const uint32_t v = cand_at(e);
        if (((v >> 18) & 4095) == (uint32_t)c1) atomicAdd(&bins2[(v >> 10) & 255], 1);
      }
      __syncthreads();
      const int hb2[1] = {tid < 256 ? bins2[tid] : 0};
      int c2, above2;
      fu_find_bin<1>(hb2, need, scr, &c2, &above2);
      tlow = ((uint32_t)c1 << 8) | (uint32_t)c2;
      room = max(need - above2, 0);
    }
    T = ((uint32_t)c0 << 20) | tlow;
    // per workgroup: its candidates above T (which join its bitmap now) and equal to T, summed over the block's 16
    // threads
    for (int e = q; e < nc; e += 16) {
      const uint32_t v = e == q ? cq : cand_at(e);
      gt += (v >> 10) > tlow;
      eq += (v >> 10) == tlow;
      if ((v >> 10) > tlow) atomicOr(&sb[FU_BMW * w + ((v & 1023u) >> 5)], 1u << (v & 31u));
    }
    gt = row_sum(gt);
    eq = row_sum(eq);
  }
  if (q == 0) {
    st.gt[w] = gt;
    st.eq[w] = eq;
  }
  __syncthreads();
  // every wave: per workgroup w (lane w) the ties at T before it, its selected count and first output index (ties
  // are taken while fewer than `room` come before, so w selects na + gt + its ties taken)
  const int eqw = lane < FU_NW ? st.eq[ww] : 0;
  const int tbw = wave_incl_scan(eqw) - eqw;
  const int selw = lane < FU_NW ? nav + st.gt[ww] + min(max(room - tbw, 0), eqw) : 0;
  const int offw = wave_incl_scan(selw) - selw;
  const int cnt_row = min(st.nvis, a.keep);
  // the ties at T taken join their block's bitmap: ties are taken while fewer than `room` ties of the row come
  // before, so a block takes all its ties, none, or (the one block where the room runs out) the first room - TB in
  // candidate order, which is position order (counted across its 16 threads)
  if (c0 >= 0) {
    const uint32_t tlow = T & 0xFFFFFu;
    const int TB = __shfl(tbw, w, WAVE), EQ = __shfl(eqw, w, WAVE);
    if (EQ > 0 && TB < room) {  // uniform over the block's 16 threads
      int ties = 0;  // the block's ties in the rounds before
      for (int e0 = 0; e0 < nc; e0 += 16) {
        const int e = e0 + q;
        const uint32_t v = e < nc ? (e0 == 0 ? cq : cand_at(e)) : 0u;
        const bool tie = e < nc && (v >> 10) == tlow;
        const int incl = row_incl_scan(tie);  // the block's ties up to this one in the round
        if (tie && TB + ties + incl - 1 < room) atomicOr(&sb[FU_BMW * w + ((v & 1023u) >> 5)], 1u << (v & 31u));
        ties += row_sum(tie);
      }
    }
  }
  __syncthreads();
  return fu_split_slots<HPW>(a, lds, b, j, kw, selw, offw, o0, o1, cnt_row, pg0, qv, live_bias);
}

// Stages 2 and 3 in one exchange, from the key lists: every workgroup reads all 32 lists of the row (thread (w, q):
// list w's entries FU_LPT q .. + FU_LPT - 1) and the row's pages. Every key of the row at or above the lowest bin of
// each list is in the lists, so when the bin c0 of the lists' keep-th largest key is at or above every list's lowest
// bin, the lists hold every key at or above the row's keep-th largest, and T (the keep-th largest), the ties at T to
// take (the lowest positions) and every selected key's index in the ascending output follow from the lists alone
// (three histogram passes over their keys: 12, 12 and 8 bits; then per list its counts above and at T): the
// workgroup writes the indices and lists the cache slots of its split's outputs [o0, o1) straight from its listed
// keys. Returns false when the lists do not hold the selection (every workgroup of the row decides alike, and nothing
// but LDS has been written): the caller then takes the two-exchange form. The pooled form (POOL: every list holds its
// whole block, so this never returns false) selects pools: each selected pool in the split lists its kpool token
// slots, and the split holding the row's last selected pool (split 0 when none is) lists the row's tail tokens
// kpool npool .. position after them (trnrt/models/dsa_long.py:189-215, the masked slots left out).
template <int HPW, bool POOL = false>
__device__ __forceinline__ bool fu_select_lists(const FusedArgs& a, uint8_t* lds, int b, int j, int L,
                                                u32x4 (&qv)[FuAtt<HPW, POOL ? 512 : FU_DQK, POOL>::QPT],
                                                float* live_bias, int* n_slots) {
  constexpr int DQK = POOL ? 512 : FU_DQK;
  using AT = FuAtt<HPW, DQK, POOL>;
  using FF = FuForm<POOL>;
  constexpr int QPT = AT::QPT, LPT = FF::LPT;
  FuState& st = *reinterpret_cast<FuState*>(lds + L_STATE);
  int* bins0 = reinterpret_cast<int*>(lds + L_CB);
  int* bins1 = reinterpret_cast<int*>(lds + L_BINS);
  int* bins2 = reinterpret_cast<int*>(lds + L_BINS2);
  int* co0 = reinterpret_cast<int*>(lds + L_CO0);
  int* co1 = reinterpret_cast<int*>(lds + L_CO1);
  int* spg = reinterpret_cast<int*>(lds + L_SPG);
  int* slot_l = reinterpret_cast<int*>(lds + AT::L_P);
  // the split's output positions, stored to idx in one coalesced pass at the end; the entry past SPLIT is the sink
  // for the writes of entries outside the split
  constexpr int POS_SINK = AT::SPLIT;
  int* pos_l = slot_l + AT::CAP + 8;
  static_assert(4 * (AT::CAP + 8 + AT::SPLIT + 1) <= 2 * HPW * AT::PROW, "slot and position lists inside P's region");
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int w = tid >> 4, q = tid & 15;
  const int hg = j % a.HG, s = j / a.HG;
  const bool active = s < a.S;  // workgroup-uniform: a workgroup past the last split only helps with the barriers
  const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
  // list w's counts and this thread's entries (plain buffer loads: the lists are the peers' stores, in lines of their
  // own that no workgroup read before barrier A); the pooled form: the list's keys LPT q .. LPT q + 15 and its
  // header bins 4 q .. 4 q + 3
  constexpr int NL = POOL ? LPT / 4 : LPT / 2;
  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.lst + (size_t)b * FU_NW * FF::LROW), (short)0, FU_NW * FF::LROW * 4, FU_BUF_WORD3);
  const int lo = 4 * FF::LROW * w;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  uint32_t hw0 = 0u, hw1 = 0u;
  u32x2 hp = {0u, 0u};
  u32x4 bh = {0u, 0u, 0u, 0u};
  if constexpr (!POOL) {
    hw0 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(lrs, lo, 0, FU_AUX_PLAIN);
    hw1 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(lrs, lo + 4, 0, FU_AUX_PLAIN);
    // header bins 2 q, 2 q + 1 (threads q < 14)
    hp = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(lrs, lo + 16 + 8 * min(q, FU_LBINS / 2 - 1), 0, FU_AUX_PLAIN));
  } else {
    // header entries 4 q .. 4 q + 3
    bh = __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(lrs, lo + 4 * FF::LCAP + 16 * q, 0, FU_AUX_PLAIN));
  }
  u32x4 ev[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i)
    ev[i] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                   lrs, POOL ? lo + 4 * LPT * q + 16 * i : lo + 4 * FU_LHDR + 8 * LPT * q + 16 * i, 0, FU_AUX_PLAIN));
  __builtin_amdgcn_sched_barrier(0);
  // the row's pages into registers (pages tid, tid + 512, clamped: at most 1024 pages of at least 32 tokens), staged
  // in LDS at the end (loads straight into LDS here would make every LDS access below wait for all loads, the
  // queries' included)
  int pgv[2];
  {
    const int* trow = a.table + (size_t)b * a.max_pages;
    // (pooled: the pages of pools 0 .. L, the last the tail pool's)
    const int npg = POOL ? (L >> a.ppp_shift) + 1 : (L + a.page_size - 1) >> a.page_shift;
#pragma unroll
    for (int c = 0; c < 2; ++c) pgv[c] = trow[max(min(min(tid + FU_THREADS * c, npg - 1), a.max_pages - 1), 0)];
  }
  __builtin_amdgcn_sched_barrier(0);
  {
    // (unconditional: a workgroup past the last split loads its head group's queries and never uses them, and no
    // register copy of a query waits for its load at a join)
    const u32x4* qsrc = reinterpret_cast<const u32x4*>(a.q + ((size_t)b * a.H + HPW * hg) * DQK);
#pragma unroll
    for (int i = 0; i < QPT; ++i) qv[i] = qsrc[min(tid + FU_THREADS * i, HPW * DQK / 8 - 1)];
  }
  const int kw = fu_kw(L);
  fu_store_scores(a, lds, b, j, kw);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = tid; i < 4096; i += FU_THREADS) bins0[i] = bins1[i] = 0;
  if (tid < 256) bins2[tid] = 0;
  if (tid < 64) co0[tid] = co1[tid] = 0;
  if (tid < AT::CAP) slot_l[tid] = 0;  // padding rows read slot 0
  if (tid < AT::SPLIT) pos_l[tid] = 0;  // outputs past the count are 0
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the bins cleared (the loads above may be out; their first uses wait for them)
  uint32_t key[LPT], pos[LPT];
  if constexpr (POOL) {
    // the block's keys LPT q + i (those at kw and past are not the block's)
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      key[i] = LPT * q + i < kw ? ev[i / 4][i & 3] : 0u;
      pos[i] = (uint32_t)(LPT * q + i);
    }
  } else {
    const int nw = min((int)hw0, FF::LCAP) - LPT * q;  // this thread's entries: those below nw
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      key[i] = i < nw ? ev[i / 2][2 * (i & 1)] : 0u;
      pos[i] = ev[i / 2][2 * (i & 1) + 1] & 1023u;
    }
  }
  // the keys pass through an empty asm between the passes below, so that no compare mask over them is kept across
  // passes (twelve 64-bit masks held in scalar registers spill)
  auto fresh = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) asm volatile("" : "+v"(key[i]));
  };
  // a histogram level's counts go to its 4096 bins and their 64 coarse bins (the wave-level bin searches below read
  // both after one barrier)
  // (the first level's coarse bins are summed from the fine ones after the adds: the lists' header bins are the
  // highest, so their coarse bins are few, and adding to them directly queued thousands of atomics on a few words)
  auto add0 = [&](uint32_t bin, int n) __attribute__((always_inline)) { atomicAdd(&bins0[bin], n); };
  int c0, above0, nlist, cnt_row;
  if constexpr (POOL) {
    // the first level from the lists' headers: exact for the bins at or above every list's lowest complete bin lmax
    // (a list's 64th header bin when it has one, else every bin); when the keep-th largest key's bin c0 is below
    // that, the keys below their list's header bins are counted one by one and the search repeated
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (bh[k]) add0((bh[k] >> 16) & 4095u, (int)(bh[k] & 0xFFFFu));
    if (q == 15) st.lbin[w] = bh[3] ? (int)(bh[3] >> 16) : 0;
    __syncthreads();
    fu_coarse_sums(bins0, co0);
    __syncthreads();
    nlist = fu_wave_find(bins0, co0, a.keep, &c0, &above0);
    const int lmax = (int)wave_max_u32(lane < FU_NW ? (uint32_t)st.lbin[lane] : 0u);
    if (lmax > 0 && (nlist <= a.keep || c0 < lmax)) {  // workgroup-uniform
      const int low = st.lbin[w];
      __syncthreads();  // every wave's search above has read the bins
#pragma unroll
      for (int i = 0; i < LPT; ++i)
        if (key[i] && (int)(key[i] >> 20) < low) add0(key[i] >> 20, 1);
      fresh();
      __syncthreads();
      fu_coarse_sums(bins0, co0);
      __syncthreads();
      nlist = fu_wave_find(bins0, co0, a.keep, &c0, &above0);
    }
    // every list holds all its workgroup's keys
    cnt_row = min(nlist, a.keep);
    if (nlist <= a.keep) c0 = -1;  // every selectable key is selected
  } else {
    // the first level from the lists' header bins (their bins at or above the lowest listed are exactly the listed
    // keys' bins); a list whose 28th header bin is listed may list more bins than its header holds: its keys one by
    // one
    const bool hfull = q == FU_LBINS / 2 - 1 && hp[1] != 0u && (hp[1] >> 16) >= hw1;
    if ((__ballot(hfull) >> (16 * (w & 3))) & 0xFFFFull) {
#pragma unroll
      for (int i = 0; i < LPT; ++i)
        if (key[i]) add0(key[i] >> 20, 1);
    } else if (q < FU_LBINS / 2) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (hp[k] != 0u && (hp[k] >> 16) >= hw1) add0((hp[k] >> 16) & 4095u, (int)(hp[k] & 0xFFFFu));
    }
    fresh();
    if (q == 0) st.lbin[w] = (int)hw1;
    __syncthreads();
    fu_coarse_sums(bins0, co0);
    __syncthreads();
    nlist = fu_wave_find(bins0, co0, a.keep, &c0, &above0);
    const uint32_t lmax = wave_max_u32(lane < FU_NW ? (uint32_t)st.lbin[lane] : 0u);
    if (lmax == 0u) {
      // every list holds all its workgroup's keys
      cnt_row = min(nlist, a.keep);
      if (nlist <= a.keep) c0 = -1;  // every selectable key is selected
    } else {
      if (nlist < a.keep || c0 < (int)lmax) return false;
      cnt_row = a.keep;
    }
  }
  // T and the room for ties at T; with c0 = -1, T = 0 (below every listed key) and no ties
  uint32_t T = 0u;
  int room = 0;
  if (c0 >= 0) {
#pragma unroll
    for (int i = 0; i < LPT; ++i)
      if (key[i] && (int)(key[i] >> 20) == c0) atomicAdd(&bins1[(key[i] >> 8) & 4095u], 1);
    fresh();
    __syncthreads();
    fu_coarse_sums(bins1, co1);  // (as the first level's: a pooled row's bin c0 can hold hundreds of keys)
    __syncthreads();
    int c1, above1;
    int need = a.keep - above0;
    fu_wave_find(bins1, co1, need, &c1, &above1);
    need -= above1;
    uint32_t tlow;
    if (need >= bins1[c1]) {
      // every key of bin c1 is taken: T is the bin's lowest key, and all its ties
      tlow = (uint32_t)c1 << 8;
      room = need;
    } else {
      const uint32_t hi24 = ((uint32_t)c0 << 12) | (uint32_t)c1;
#pragma unroll
      for (int i = 0; i < LPT; ++i)
        if (key[i] && (key[i] >> 8) == hi24) atomicAdd(&bins2[key[i] & 255u], 1);
      fresh();
      __syncthreads();
      int c2, above2;
      fu_wave_find256(bins2, need, &c2, &above2);
      tlow = ((uint32_t)c1 << 8) | (uint32_t)c2;
      room = max(need - above2, 0);
    }
    T = ((uint32_t)c0 << 20) | tlow;
  }
  // every listed key's place in the ascending output, from the lists alone: per list, its keys above T and its ties
  // at T (packed counts, summed over its 16 threads in list order); then per list the ties of the lists before it
  // (ties are taken in position order while fewer than `room` come before), its selected count and its first output
  // index; a selected key's index is its list's first plus the selected keys before it in the list
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < LPT; ++i) mine += (key[i] > T ? 1u : 0u) + (key[i] == T && key[i] ? 0x10000u : 0u);
  fresh();
  const uint32_t incl = (uint32_t)row_incl_scan((int)mine);
  if (q == 15) {
    st.gt[w] = (int)(incl & 0xFFFFu);
    st.eq[w] = (int)(incl >> 16);
  }
  spg[tid] = pgv[0];
  spg[tid + FU_THREADS] = pgv[1];
  __syncthreads();
  const int ww = lane & (FU_NW - 1);
  const int eqw = lane < FU_NW ? st.eq[ww] : 0;
  const int tbw = wave_incl_scan(eqw) - eqw;
  const int takew = lane < FU_NW ? min(max(room - tbw, 0), eqw) : 0;  // list w's ties taken: its first takew
  const int selw = lane < FU_NW ? st.gt[ww] + takew : 0;
  const int offw = wave_incl_scan(selw) - selw;
  // (with every lane active: a lane switched off returns no value)
  const int off_l = __shfl(offw, w, WAVE), take_l = __shfl(takew, w, WAVE);
  // the attention's queries into LDS before the index stores below (a wait for the queries' loads there would also
  // wait for those stores)
  {
    uint16_t* qs = reinterpret_cast<uint16_t*>(lds + AT::L_QST);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int pc = tid + FU_THREADS * i;
      if (active && pc < HPW * DQK / 8)
        *reinterpret_cast<u32x4*>(qs + (pc / (DQK / 8)) * AT::AQROW + 8 * (pc % (DQK / 8))) = qv[i];
    }
  }
  {
    // this thread's selected entries take the output indices first .. first + nsel - 1; only the threads whose
    // indices meet the split's [o0, o1) (one or two lists' worth, so most waves skip this) store their entries'
    // positions, with no branch per entry (an entry outside the split writes the sink entry past the list); the
    // cache slots follow from the positions below, one thread per slot
    int gtb = (int)((incl - mine) & 0xFFFFu), eqb = (int)((incl - mine) >> 16);  // this thread's list predecessors
    const int first = off_l + gtb + min(eqb, take_l);
    const int nsel = (int)(mine & 0xFFFFu) + min(max(take_l - eqb, 0), (int)(mine >> 16));
    if (nsel > 0 && first < o1 && first + nsel > o0) {
      const int nties = (int)(mine >> 16);
      if (nties == 0 || eqb >= take_l || eqb + nties <= take_l) {
        // none of this thread's ties is taken, or all are (every thread but at most one of the row): its selected
        // entries are those at or above one threshold (T + 1 or T; T >= 1 when there are ties)
        const uint32_t thr = nties > 0 && eqb < take_l ? T : T + 1u;
        int r = first - o0;  // the next selected entry's output index in the split
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
          const bool sl = key[i] >= thr;
          pos_l[sl && (unsigned)r < (unsigned)(o1 - o0) ? r : POS_SINK] = kw * w + (int)pos[i];
          r += sl;
        }
      } else {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
          const bool above = key[i] > T, tie = key[i] == T && key[i];
          const int o = off_l + gtb + min(eqb, take_l) - o0;
          const bool in = (above || (tie && eqb < take_l)) && (unsigned)o < (unsigned)(o1 - o0);
          pos_l[in ? o : POS_SINK] = kw * w + (int)pos[i];  // the key's position (pooled: pool) in the row
          gtb += above;
          eqb += tie;
        }
      }
    }
  }
  if (j == 0 && tid == 0) a.cnt[b] = cnt_row;
  // the split's live slots; a row with none attends position 0 masked (its lse is NEG_INF)
  int ns = max(min(o1, cnt_row) - o0, 0);
  bool empty = cnt_row == 0;
  __syncthreads();  // the split's positions
  if (POOL) {
    // the selected pools' token slots (token t & (kpool - 1) of the split's pool t >> log2 kpool: consecutive slots
    // of its page), then (in the split of the last selected pool) the tail's: tokens kpool L .. position of the
    // incomplete pool L, in that pool's page
    ns <<= a.kp_shift;
    if (tid < ns) {
      const int p = pos_l[tid >> a.kp_shift];
      slot_l[tid] = safe_page(spg[p >> a.ppp_shift], a.num_pages) * a.page_size +
                    ((p & ((1 << a.ppp_shift) - 1)) << a.kp_shift) + (tid & ((1 << a.kp_shift) - 1));
    }
    const int tail_pos0 = L << a.kp_shift;
    const int tail = min(max(a.positions[b] + 1 - tail_pos0, 0), (1 << a.kp_shift) - 1);
    const int s_last = cnt_row > 0 ? (cnt_row - 1) / a.sps : 0;
    if (active && s == s_last && tail > 0) {
      if (tid < tail)
        slot_l[ns + tid] = safe_page(spg[L >> a.ppp_shift], a.num_pages) * a.page_size +
                           ((tail_pos0 + tid) & (a.page_size - 1));
      ns += tail;
    }
    empty = cnt_row == 0 && tail == 0;
  } else if (tid < ns) {
    const int p = pos_l[tid];
    slot_l[tid] = safe_page(spg[p >> a.page_shift], a.num_pages) * a.page_size + (p & (a.page_size - 1));
  }
  *live_bias = 0.0f;
  if (active && empty && s == 0) {
    ns = 1;
    *live_bias = NEG_INF;
    if (tid == 0) slot_l[0] = safe_page(a.table[(size_t)b * a.max_pages], a.num_pages) * a.page_size;
  }
  *n_slots = ns;
  __syncthreads();  // the slot and position lists and the queries
  // the split's outputs [o0, o1) of the ascending index output, one coalesced store (0 past the count)
  if (hg == 0 && tid < o1 - o0) a.idx[(size_t)b * a.keep + o0 + tid] = pos_l[tid];
  return true;
}

// The value operand of v_mfma_f32_16x16x32_bf16 from the token-major tile (ds_read_b64_tr_b8: lane (a, c) of each
// 16-lane block gets byte c of the 8-byte rows addressed by the block's lanes 2j + a): lane l receives dim 16 n + l % 16
// of tokens 32 ks + 8 (l / 16) + j, the B operand with k-slot 8 q + j = that token.
template <int KROW>
__device__ __forceinline__ bf16x8 fu_value_operand(const uint8_t* kt, int ks, int n, int lane) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const int q = lane >> 4, p = lane & 15;
  const uint8_t* ad = kt + (32 * ks + 8 * q + (p >> 1)) * KROW + 16 * n + 8 * (p & 1);
  const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(ad));
  return fp8x8_to_bf16x8((uint32_t)r.x, (uint32_t)r.y);
}

// Stage 4: the split's attention over the n_slots slots of the list at FuAtt<HPW, DQK, XT>::L_P (at most CAP), with
// the queries staged before at qoff. gather = false: the rows, their scales and biases are still in LDS from the
// previous call over the same slots (queries past the row tile only), and the slot list is not read.
template <int HPW, int DQK = FU_DQK, bool XT = false>
__device__ __forceinline__ void fu_attend(const FusedArgs& a, uint8_t* lds, int b, int j, int n_slots,
                                          float live_bias, bool gather = true, int qoff = FuAtt<HPW, DQK, XT>::L_QST) {
  using AT = FuAtt<HPW, DQK, XT>;
  constexpr int HB = AT::HB, TG = AT::TG, PROW = AT::PROW, KROW = AT::KROW, KPIECES = AT::KPIECES;
  constexpr int PIECES = AT::PIECES, STEPS = AT::STEPS, AQROW = AT::AQROW;
  float* ksc_l = reinterpret_cast<float*>(lds + AT::L_KSC);
  float* bias_l = reinterpret_cast<float*>(lds + AT::L_BIAS);
  float* red = reinterpret_cast<float*>(lds + AT::L_RED);
  float* sred = reinterpret_cast<float*>(lds + AT::L_SRED);
  uint16_t* pl = reinterpret_cast<uint16_t*>(lds + AT::L_P);
  uint8_t* kt = lds + L_KT;
  const uint16_t* qs = reinterpret_cast<const uint16_t*>(lds + qoff);
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid & (WAVE - 1);
  const int l16 = lane & 15, q4 = lane >> 4;
  const int hb = wave % HB, tg = wave / HB;  // the scores: this wave's 16-head block and 32-token group
  const int hg = j % a.HG, s = j / a.HG;
  if (s >= a.S) return;  // workgroup-uniform
  const int H = a.H;
  // head HPW hg + i's split output at part + i * 512, its (max, sum) at mlp[i] (the split's pairs [S][H]: each
  // workgroup's in whole 128-byte lines of its own)
  uint16_t* part = a.part + (((size_t)b * a.S + s) * H + HPW * hg) * FU_DV;
  float2* mlp = a.ml + ((size_t)b * a.S + s) * H + HPW * hg;
  if (n_slots == 0) {  // an empty split: weight 0 in the combine
    for (int i = tid; i < HPW * FU_DV / 8; i += FU_THREADS)
      reinterpret_cast<uint4*>(part + (size_t)(i / (FU_DV / 8)) * FU_DV)[i % (FU_DV / 8)] = uint4{0u, 0u, 0u, 0u};
    if (tid < HPW) mlp[tid] = make_float2(-INFINITY, 0.0f);
    return;
  }
  static_assert(FU_CH * KPIECES % WAVE == 0 && AT::CAP % FU_CH == 0, "a padded split's pieces fill whole loads");
  const int padded = (n_slots + FU_CH - 1) / FU_CH * FU_CH;

  // the slot list (a padding row reads slot 0) and the queries (staged in LDS by stage 3)
  const int* slot_l = reinterpret_cast<const int*>(lds + AT::L_P);
  const int slot = tid < AT::CAP ? slot_l[tid] : 0;
  // the query operand: head 16 hb + l16, dims 64 (st / 2) + 16 q4 + 8 (st % 2) .. + 7 at score step st (the key
  // operand's dim order below)
  bf16x8 qb[STEPS];
  {
    const uint16_t* qh = qs + (16 * hb + l16) * AQROW + 16 * q4;
#pragma unroll
    for (int st2 = 0; st2 < STEPS; ++st2)
      qb[st2] = as_bf16x8(*reinterpret_cast<const uint4*>(qh + 64 * (st2 >> 1) + 8 * (st2 & 1)));
  }
  // (16 heads: the queries are staged inside the row tile, so every wave holds its query operand before the rows
  // overwrite it; 32: they lie past the tile, and the gather below starts while the operand reads are in flight)
  if (AT::L_QST < AT::L_P) __syncthreads();
  // every row straight into LDS, coalesced: load k fills 1 KiB of the tile, lane l 16-byte unit u = 64 k + l (row
  // u / 37, piece u % 37; the padding piece re-reads the last data piece); the loads of the padded rows' units spread
  // over the 8 waves
  if (gather) {
    // unit u = 64 k + lane's row u / 37 and piece u % 37, advanced with k (by 8: u by 512 = 13 x 37 + 31); the
    // lane's slots for its loads k = wave + 8 i in one round of LDS reads, then the loads (a slot read per load
    // would put an LDS round trip before each)
    constexpr int DR = FU_WAVES * WAVE / KPIECES, DP = FU_WAVES * WAVE % KPIECES;
    constexpr int NI = (AT::CAP * KPIECES + FU_THREADS - 1) / FU_THREADS;  // loads per lane at most
    const int units = padded * KPIECES;
    const int row0 = (WAVE * wave + lane) / KPIECES, pc0 = WAVE * wave + lane - row0 * KPIECES;
    int row = row0, pc = pc0;
    int sl[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      sl[i] = slot_l[min(row, AT::CAP - 1)];  // (past the units: a row of the list, never loaded)
      row += DR;
      pc += DP;
      if (pc >= KPIECES) {
        pc -= KPIECES;
        ++row;
      }
    }
    pc = pc0;  // (the pieces again, stepped as above)
    // (opaque here: in a kernel that attends several rows in turn, the loads' per-lane offsets would otherwise be
    // computed once before the rows and held in registers throughout, which spills)
    asm volatile("" : "+v"(pc));
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int k = wave + FU_WAVES * i;
      if (k * WAVE < units) {
        const uint8_t* src = a.kv + (size_t)sl[i] * DQK + 16 * min(pc, PIECES - 1);
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(kt + 1024 * k), 16, 0, 0);
      }
      pc += DP;
      if (pc >= KPIECES) pc -= KPIECES;
    }
  }
  if (gather) {
    const float ksv = tid < padded ? (a.kvs ? a.kvs[slot] : 1.0f) : 0.0f;  // kvs null: the unscaled cache
    __builtin_amdgcn_s_waitcnt(0);
    if (tid < padded) {
      ksc_l[tid] = ksv;
      bias_l[tid] = tid < n_slots ? live_bias : -INFINITY;
    }
  }
  __syncthreads();  // every row in LDS

  // scores of tokens 32 g .. + 31 (two blocks of 16) for heads 16 hb .. + 15, g = tg and (XT, tg < 2) tg + TG:
  // S^T = K . Q^T;
  // lane group q4 reads piece 4 j + q4 (dims 64 j + 16 q4 ..) of its token per pair of steps (one ds_read_b128 for two
  // MFMAs; 8 rows at one column cover the banks once at the row stride)
  auto scores_of = [&](int g, float (&sv)[2][4], float& mx) __attribute__((always_inline)) {
    f32x4 acc[2][2];
#pragma unroll
    for (int k = 0; k < 2; ++k) acc[k][0] = acc[k][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint8_t* kr = kt + (32 * g + l16) * KROW + 16 * q4;
#pragma unroll
    for (int st2 = 0; st2 < STEPS; st2 += 2) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const u32x4 kk = *reinterpret_cast<const u32x4*>(kr + 16 * k * KROW + 32 * st2);
        acc[k][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[0], kk[1]), qb[st2], acc[k][0], 0, 0, 0);
        acc[k][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(kk[2], kk[3]), qb[st2 + 1], acc[k][1], 0, 0,
                                                            0);
      }
    }
    // acc[k][.][r] = S^T[token 32 g + 16 k + 4 q4 + r][head 16 hb + l16]
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int tk = 32 * g + 16 * k + 4 * q4;
      const float4 ks4 = *reinterpret_cast<const float4*>(&ksc_l[tk]);
      const float4 bs4 = *reinterpret_cast<const float4*>(&bias_l[tk]);
      sv[k][0] = (acc[k][0][0] + acc[k][1][0]) * (ks4.x * a.scale) + bs4.x;
      sv[k][1] = (acc[k][0][1] + acc[k][1][1]) * (ks4.y * a.scale) + bs4.y;
      sv[k][2] = (acc[k][0][2] + acc[k][1][2]) * (ks4.z * a.scale) + bs4.z;
      sv[k][3] = (acc[k][0][3] + acc[k][1][3]) * (ks4.w * a.scale) + bs4.w;
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = max_nonan(mx, sv[k][i]);
    }
  };
  const bool has = 32 * tg < padded;
  const bool has2 = XT && 32 * (tg + TG) < padded;  // the tail's rows past the split's TG groups (tg < 2: CAP)
  float sv[2][4], sx[2][4];
  float mx = -INFINITY;
  if (has) scores_of(tg, sv, mx);
  if (has2) scores_of(tg + TG, sx, mx);
  mx = max_nonan(mx, __shfl_xor(mx, 16, WAVE));
  mx = max_nonan(mx, __shfl_xor(mx, 32, WAVE));
  if (lane < 16) red[(16 * hb + lane) * TG + tg] = mx;
  __syncthreads();
  float m = -INFINITY;
  {
    float r[TG];  // head 16 hb + l16's maxima over the token groups, in one or two vector reads
#pragma unroll
    for (int t = 0; t < TG; t += 4)
      *reinterpret_cast<float4*>(r + t) = *reinterpret_cast<const float4*>(&red[(16 * hb + l16) * TG + t]);
#pragma unroll
    for (int t = 0; t < TG; ++t) m = max_nonan(m, r[t]);
  }
  float psum = 0.0f;
  // the weights of group g: exp(s - m), the value's dequantisation folded into the bf16 weight
  auto weights_of = [&](int g, const float (&sv)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int tk = 32 * g + 16 * k + 4 * q4;
      const float4 ks4 = *reinterpret_cast<const float4*>(&ksc_l[tk]);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __expf(sv[k][i] - m);
        psum += p[i];
      }
      *reinterpret_cast<uint2*>(&pl[(16 * hb + l16) * PROW + tk]) =
          make_uint2(bf16_pack(p[0] * ks4.x, p[1] * ks4.y), bf16_pack(p[2] * ks4.z, p[3] * ks4.w));
    }
  };
  if (has) weights_of(tg, sv);
  if (has2) weights_of(tg + TG, sx);
  psum += __shfl_xor(psum, 16, WAVE);
  psum += __shfl_xor(psum, 32, WAVE);
  if (lane < 16) sred[(16 * hb + lane) * TG + tg] = psum;
  __syncthreads();  // P and the sums

  // O[heads][dims 64 wave ..] += P . V over the split's tokens, the value operand shared by the HB head blocks
  f32x4 o[HB][4];
#pragma unroll
  for (int h = 0; h < HB; ++h)
#pragma unroll
    for (int n = 0; n < 4; ++n) o[h][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nks = padded / 32;
  for (int ks = 0; ks < nks; ++ks) {
    bf16x8 pop[HB];
#pragma unroll
    for (int h = 0; h < HB; ++h)
      pop[h] = as_bf16x8(*reinterpret_cast<const uint4*>(&pl[(16 * h + l16) * PROW + 32 * ks + 8 * q4]));
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const bf16x8 vop = fu_value_operand<KROW>(kt, ks, 4 * wave + n, lane);
#pragma unroll
      for (int h = 0; h < HB; ++h) o[h][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[h], vop, o[h][n], 0, 0, 0);
    }
  }
  // the split's output (bf16, not normalised: the combine divides by the splits' total), max and sum: lane (l16, q4)
  // holds heads 16 h + 4 q4 + i at dim 64 wave + 16 n + l16; neighbouring lanes swap halves so that an even lane
  // stores heads i = 0, 1 and an odd lane heads i = 2, 3, each as a pair of dims; wave 0's lanes l16 = 0 store the
  // (max, sum) pairs
  const bool odd = l16 & 1;
  if (wave == 0 && l16 == 0) {
#pragma unroll
    for (int h = 0; h < HB; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hl = 16 * h + 4 * q4 + i;
        float r[TG], mr[TG];
#pragma unroll
        for (int t = 0; t < TG; t += 4) {
          *reinterpret_cast<float4*>(r + t) = *reinterpret_cast<const float4*>(&sred[hl * TG + t]);
          *reinterpret_cast<float4*>(mr + t) = *reinterpret_cast<const float4*>(&red[hl * TG + t]);
        }
        float l = 0.0f, mh = -INFINITY;
#pragma unroll
        for (int t = 0; t < TG; ++t) {
          l += r[t];
          mh = max_nonan(mh, mr[t]);
        }
        mlp[hl] = make_float2(mh, l);
      }
  }
#pragma unroll
  for (int h = 0; h < HB; ++h) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = o[h][n][i];
      const float u0 = lane_xor1(odd ? v[0] : v[2]), u1 = lane_xor1(odd ? v[1] : v[3]);
      const int hl = 16 * h + 4 * q4 + (odd ? 2 : 0);
      uint16_t* ph = part + (size_t)hl * FU_DV + 64 * wave + 16 * n + (l16 & ~1);
      *reinterpret_cast<uint32_t*>(ph) = odd ? bf16_pack(u0, v[2]) : bf16_pack(v[0], u0);
      *reinterpret_cast<uint32_t*>(ph + (size_t)FU_DV) = odd ? bf16_pack(u1, v[3]) : bf16_pack(v[1], u1);
    }
  }
}

// Stage 5: the splits merged by log-sum-exp, o = sum_s W_s o_s / sum_s W_s with W_s = l_s exp(m_s - M) over the
// splits with l_s > 0 and lse = M + log sum_s W_s. Workgroup j takes heads 2 j, 2 j + 1 (then + 64, ...), thread t
// head 2 j + t / 256, dims 2 (t % 256) ..: wave 0 loads the two heads' (max, sum) pairs (lane 32 h + s for head h,
// split s), then every thread's NS split loads go out (unconditionally, a split past S re-reading the last one), wave
// 0 turns the pairs into the weights W_s / sum W in LDS (0 past S), and each thread sums its weighted dims.
template <int NS>
__device__ __forceinline__ void fu_combine_heads(const FusedArgs& a, float* wts, int b, int h0) {
  const int S = a.S, H = a.H, tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int h = h0 + (tid >> 8), d = 2 * (tid & 255);
  const int hh = h0 + (lane >> 5), sp = lane & 31;
  uint64_t mlv = 0;
  if (tid < WAVE) mlv = *reinterpret_cast<const uint64_t*>(a.ml + ((size_t)b * S + min(sp, S - 1)) * H + hh);
  // the two heads' split outputs through a buffer descriptor: split k's offset is scalar, the lane's is 32-bit
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.part + (size_t)b * S * H * FU_DV + (size_t)h0 * FU_DV), (short)0,
      2 * ((S - 1) * H * FU_DV + 2 * FU_DV), FU_BUF_WORD3);
  const int voff = 2 * ((tid >> 8) * FU_DV + d);
  uint32_t ov[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k)
    ov[k] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(prs, voff, 2 * H * FU_DV * min(k, S - 1), FU_AUX_PLAIN);
  if (tid < WAVE) {
    const float m = __uint_as_float((uint32_t)mlv), l = __uint_as_float((uint32_t)(mlv >> 32));
    const bool live = sp < S && l > 0.0f;
    float M = row_max(live ? m : -INFINITY);
    M = fmaxf(M, __shfl_xor(M, 16, WAVE));  // the two rows of the head's 32 lanes
    // split s's output is its unnormalised sum of exp(score - m_s) v: weighted by exp(m_s - M) / W, W the splits'
    // total sum at the common maximum M
    const float e = live ? __expf(m - M) : 0.0f;
    float W = row_sum(e * l);
    W += __shfl_xor(W, 16, WAVE);
    wts[lane] = e * __builtin_amdgcn_rcpf(W);  // W >= 1 (the largest split's weight is its sum)
    if (sp == 0 && a.lse) a.lse[(size_t)b * H + hh] = M + __logf(W);
  }
  __syncthreads();
  float x0 = 0.0f, x1 = 0.0f;
  const float* wh = wts + 32 * (tid >> 8);
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const float wk = wh[k];
    x0 += wk * __uint_as_float(ov[k] << 16);
    x1 += wk * __uint_as_float(ov[k] & 0xFFFF0000u);
  }
  *reinterpret_cast<uint32_t*>(a.out + ((size_t)b * H + h) * FU_DV + d) = bf16_pack(x0, x1);
  __syncthreads();  // the weights are read before the next heads' overwrite them
}

__device__ __forceinline__ void fu_combine(const FusedArgs& a, uint8_t* lds, int b, int j) {
  float* wts = reinterpret_cast<float*>(lds);  // [2][32]
  for (int h0 = 2 * j; h0 < a.H; h0 += 2 * FU_NW) {
    if (a.S <= 16)
      fu_combine_heads<16>(a, wts, b, h0);
    else
      fu_combine_heads<32>(a, wts, b, h0);
  }
}

template <int MT, int HPW>
__global__ __launch_bounds__(FU_THREADS, 1) void decode_fused_kernel(FusedArgs a) {
  __shared__ __align__(16) uint8_t lds[FU_LDS];
  const int x = blockIdx.x % FU_XCDS, j = blockIdx.x / FU_XCDS;
  const FuSync sync = fu_sync_begin(a.sync + x * WS_SYNC_WORDS, j);
  // one row per XCD and launch (rows row0 + x; a batch of more than 8 rows takes several launches, which keeps
  // each workgroup's per-lane address arithmetic out of a loop over rows, where it would be held in registers)
  const int b = a.row0 + x;
  if (b >= a.B) return;  // an XCD without a row
  const int L = min(max(a.ctx_len[b], 0), min(a.stride, FU_MAXLEN));
  fu_indexer<MT>(a, lds, b, j, L);
  fu_barrier(sync, 1);  // A: the row's scores, histogram and key lists
  u32x4 qv[FuAtt<HPW>::QPT];
  float live_bias;
  int n_slots, nbar = 2;
  const bool lists = fu_lists_on(a, L);
  bool one = false;
  if (lists) {
    one = fu_select_lists<HPW>(a, lds, b, j, L, qv, &live_bias, &n_slots);
    if (!one) __syncthreads();  // every thread has read the bin search's results before stage 2 reuses its words
  }
  if (!one) {
    fu_classify(a, lds, b, j);
    fu_barrier(sync, 2);  // B: every workgroup's counts and candidates
    n_slots = fu_select<HPW>(a, lds, b, j, L, qv, &live_bias);
    nbar = 3;
  }
  fu_attend<HPW>(a, lds, b, j, n_slots, live_bias);
  fu_barrier(sync, nbar);  // C: every split's output
  fu_combine(a, lds, b, j);
  // the count of rows that took the two-exchange selection (here, where no later wait is held up by its round trip)
  if (nbar == 3 && j == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_add(sync.w + WS_SYNC_TWO_EXCHANGE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  fu_exit(sync, nbar);
}

// The pooled (GLM, kpool > 1) decode layer step in one launch (trnrt/models/mla.py:505-526 `attention_long` for a
// decode batch, trnrt/kernels/dsa_shell.py:2114-2321 `select2` and trnrt/kernels/dsa_satwf.py:1-20 for the served
// form): row b of rows row0 .. row0 + 7 on XCD b % 8, its npool[b] complete pools (at most 8,192) scored from the
// bf16 pool-key cache in blocks of at most 256 pools, the exact top-keep pools from the key lists (each holding its
// whole block), then the attention over the selected pools' tokens and the row's tail (512-wide rows, 32 heads a
// workgroup, splits of 128 token slots) and the combine, as the kpool-1 layer.
template <int HPW, bool WRITE>
__global__ __launch_bounds__(FU_THREADS, 1) void decode_pooled_fused_kernel(FusedArgs a) {
  __shared__ __align__(16) uint8_t lds[FU_LDS];
  const int x = blockIdx.x % FU_XCDS, j = blockIdx.x / FU_XCDS;
  const FuSync sync = fu_sync_begin(a.sync + x * WS_SYNC_WORDS, j);
  const int b = a.row0 + x;
  if (b >= a.B) return;  // an XCD without a row
  const int L = min(max(a.ctx_len[b], 0), min(a.stride, FU_POOL_MAXLEN));
  fu_indexer<1, true, WRITE>(a, lds, b, j, L);
  fu_barrier(sync, 1);  // A: the row's scores and key lists
  u32x4 qv[FuAtt<HPW, 512, true>::QPT];
  float live_bias;
  int n_slots;
  fu_select_lists<HPW, true>(a, lds, b, j, L, qv, &live_bias, &n_slots);  // (the lists hold every key)
  fu_attend<HPW, 512, true>(a, lds, b, j, n_slots, live_bias);
  fu_barrier(sync, 2);  // C: every split's output
  fu_combine(a, lds, b, j);
  fu_exit(sync, 2);
}

// The split's slot list when the selection came from the separate kernels: output positions o0 .. o1 - 1 of row b,
// as cache rows (rows [B, keep], the top-k's slot output) or as positions (idx [B, keep]) through the page table;
// the attention's queries staged in LDS as stage 2 stages them. Returns the split's selected count (the empty row:
// output 0, masked, as stage 2). The pooled form (XT; trnrt/models/mla.py:615-630, the kpool tokens of each selected
// pool and then the tail): token slot k is token k & (kpool - 1) of pool idx[b][k >> kp_shift] (below the selected
// pools' cnt kpool slots), and the tail, tokens kpool npool .. pos of the incomplete pool (none when pos + 1 is a
// multiple of kpool), follows in the split holding the last selected token (split 0 when no pool is selected).
template <int HPW, int DQK = FU_DQK, bool XT = false>
__device__ __forceinline__ int fu_attend_prep(const FusedArgs& a, const int* rows, uint8_t* lds, int b, int j,
                                              float* live_bias) {
  using AT = FuAtt<HPW, DQK, XT>;
  constexpr int QPT = AT::QPT;
  int* slot_l = reinterpret_cast<int*>(lds + AT::L_P);
  const int tid = threadIdx.x;
  const int hg = j % a.HG, s = j / a.HG;
  const bool active = s < a.S;
  const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
  int cnt_row = min(max(a.cnt[b], 0), a.keep);
  int tail = 0, tail_pos0 = 0, s_last = 0;
  const int ipr = a.keep >> a.kp_shift;  // the pooled form's selected pools a row (its idx row stride)
  if (XT) {
    cnt_row = min(max(a.cnt[b], 0), ipr) << a.kp_shift;
    const int np = max(a.npool[b], 0);
    tail_pos0 = np << a.kp_shift;
    tail = min(max(a.positions[b] + 1 - tail_pos0, 0), (1 << a.kp_shift) - 1);
    s_last = cnt_row > 0 ? (cnt_row - 1) / a.sps : 0;
  }
  u32x4 qv[QPT];
  if (active) {
    const u32x4* qsrc = reinterpret_cast<const u32x4*>(a.q + ((size_t)b * a.H + HPW * hg) * DQK);
#pragma unroll
    for (int i = 0; i < QPT; ++i) qv[i] = qsrc[min(tid + FU_THREADS * i, HPW * DQK / 8 - 1)];
  }
  const int n_sel = max(min(o1, cnt_row) - o0, 0);
  const int n_tail = XT && active && s == s_last ? tail : 0;
  const bool empty = cnt_row == 0 && tail == 0;  // the row attends output 0 (position 0), masked
  const int o = o0 + tid;
  int sl = 0;
  if (XT) {
    if (tid < n_sel + n_tail || (empty && tid == 0)) {
      int pos = 0;
      if (tid < n_sel) {
        const int pool = max(a.idx[(size_t)b * ipr + (o >> a.kp_shift)], 0);
        pos = (pool << a.kp_shift) + (o & ((1 << a.kp_shift) - 1));
      } else if (!empty) {
        pos = tail_pos0 + (tid - n_sel);
      }
      const int pi = pos / a.page_size;  // pages of any multiple of kpool
      const int pg = a.table[(size_t)b * a.max_pages + min(pi, a.max_pages - 1)];
      sl = safe_page(pg, a.num_pages) * a.page_size + (pos - pi * a.page_size);
    }
  } else if (tid < AT::SPLIT && o < o1 && o < max(cnt_row, 1)) {  // the empty row lists output 0 (position 0)
    if (rows) {
      sl = rows[(size_t)b * a.keep + o];
    } else {
      const int p = max(a.idx[(size_t)b * a.keep + o], 0), pi = p / a.page_size;  // pages of any size
      const int pg = a.table[(size_t)b * a.max_pages + min(pi, a.max_pages - 1)];
      sl = safe_page(pg, a.num_pages) * a.page_size + (p - pi * a.page_size);
    }
  }
  sl = (unsigned)sl < (unsigned)a.num_slots ? sl : 0;
  if (active) {
    uint16_t* qs = reinterpret_cast<uint16_t*>(lds + AT::L_QST);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int pc = tid + FU_THREADS * i;
      if (pc < HPW * DQK / 8)
        *reinterpret_cast<u32x4*>(qs + (pc / (DQK / 8)) * AT::AQROW + 8 * (pc % (DQK / 8))) = qv[i];
    }
  }
  if (tid < AT::CAP) slot_l[tid] = sl;  // padding rows read slot 0
  int n_slots = n_sel + n_tail;
  *live_bias = 0.0f;
  if (active && empty && s == 0) {
    n_slots = 1;
    *live_bias = NEG_INF;
  }
  __syncthreads();  // the slot list and the queries
  return n_slots;
}

// The attention and combine stages of the one-launch layer as a launch of their own, after the separate kernels'
// selection (rows of any length): rows row0 + x, row0 + x + 8, ... (up to rpl of them) on XCD x, with the same
// splits and bf16 split outputs; every workgroup takes its split of each row in turn, then one XCD-local barrier,
// then the combines.
template <int HPW, int DQK = FU_DQK, bool XT = false>
__global__ __launch_bounds__(FU_THREADS, 1) void decode_attend_kernel(FusedArgs a, const int* rows, int rpl) {
  __shared__ __align__(16) uint8_t lds[FU_LDS];
  const int x = blockIdx.x % FU_XCDS, j = blockIdx.x / FU_XCDS;
  const FuSync sync = fu_sync_begin(a.sync + x * WS_SYNC_WORDS, j);
  if (a.row0 + x >= a.B) return;  // an XCD without a row
  const int nr = min(rpl, (a.B - a.row0 - x + FU_XCDS - 1) / FU_XCDS);  // this XCD's rows
  for (int r = 0; r < nr; ++r) {
    if (r) __syncthreads();  // the previous row's attention has read its LDS before the next slot list is written
    float live_bias;
    const int b = a.row0 + x + FU_XCDS * r;
    const int n_slots = fu_attend_prep<HPW, DQK, XT>(a, rows, lds, b, j, &live_bias);
    fu_attend<HPW, DQK, XT>(a, lds, b, j, n_slots, live_bias);
  }
  fu_barrier(sync, 1);  // every split's output of the XCD's rows
  for (int r = 0; r < nr; ++r) fu_combine(a, lds, a.row0 + x + FU_XCDS * r, j);
  fu_exit(sync, 1);
}

// ---- Rows longer than 32,768 tokens: the selection, the attention and the combine in one launch ----
// After the long-row indexer (indexer_decode_long_kernel: the rows' scores [B, stride] and each row's first-level
// histogram of the top 12 key bits), the rows of a launch (row0 + x + 8 r on XCD x, r < rpl) are selected and
// attended by their XCD's 32 workgroups, replacing the long top-k's three launches (chunk counts, one resolving
// workgroup per row, ordered output) and the separate attention launch:
//   1. every workgroup finds the bin c0 of the row's keep-th largest key in the row's histogram (c0 = -1, every
//      visible key, when the row has at most keep), then lists its block of the row (positions [j bw, (j + 1) bw))
//      as the (key, position) of its keys at or above c0, in position order: a block of at most 16,384 positions
//      from its scores (one round of loads), a longer one from the indexer's maxima of its 32-key tiles (the tiles
//      whose maximum is at or above c0, which alone can hold such keys, and then their scores alone); barrier (then
//      the histogram is cleared);
//   2. every workgroup reads the 32 lists: T (the keep-th largest key) from the next 12 and 8 bits of the keys in c0,
//      each list's keys above and at T, the ties taken (the lowest positions: list order, then position order) and
//      each list's first output index;
//   3. the split's outputs [o0, o1): each list holding some of them is passed once with a block prefix of its keys
//      above and at T (a selected key's output index follows), into the idx output and the split's slot list; then
//      stage 4 of the one-launch layer (fu_attend). After the XCD's rows: barrier, the combine (stage 5).
// The selection is exact (the reference's arithmetic of trnrt/kernels/dsa_topk.py, ties to the lowest positions),
// as the long top-k's: same T, same outputs in the same order.
struct LongAttArgs {
  int* hist;          // [B][4096]: the rows' first-level histograms, zero again after the launch
  const float* tmax;  // [B][ntile]: the maxima of the rows' 32-key tiles (tile t: positions 32 t .. 32 t + 31), or
                      // null: stage 1 over the scores
  uint32_t* lst;      // [B][32][LA_HDR + 2 bw]: per workgroup its block's list
  int bw;             // positions per block, a multiple of 4,096 (at most LA_SCAN_MAX without tmax)
  int ntile;          // tiles per row of tmax, a multiple of 4
  int rpl;            // rows per XCD
};
constexpr int LA_HDR = 32;   // list header words (the count; the row's boundary bin, keys above it, visible keys)
constexpr int LA_MAXLEN = FU_NW * 65536;  // 2,097,152 tokens a row
constexpr int L_LA = 0;      // stage 2's per-list words [6][32] (L_STATE's place, before L_CO1)
static_assert(L_LA + 4 * 6 * FU_NW <= L_CO1, "the per-list words clear of the coarse bins");
// stage 1 over the scores (blocks of at most LA_SCAN_MAX positions: at most one round of loads)
constexpr int LA_PASS = 8;   // positions per thread and pass (two 16-byte score loads)
constexpr int LA_BATCH = 4;  // passes a round of loads
constexpr int LA_SCAN_MAX = LA_BATCH * FU_THREADS * LA_PASS;
constexpr int L_LA_STAGE = 81920;  // the scores [LA_BATCH][4096] (past the split's positions, dead by stage 3)
static_assert(L_LA_STAGE + LA_BATCH * FU_THREADS * LA_PASS * 4 <= FU_LDS, "stage 1's scores in LDS");
static_assert(L_LA_STAGE >= FuAtt<32>::L_P + 4 * (FuAtt<32>::CAP + 8 + FuAtt<32>::SPLIT + 1) &&
                  L_LA_STAGE + LA_BATCH * FU_THREADS * LA_PASS * 4 <= FuAtt<16>::L_P,
              "stage 1's scores clear of the split's slot and position lists");
static_assert(L_BINS + 4 * 4096 <= L_LA_STAGE, "stage 1's scores clear of the bins");
// stage 1 over the tile maxima (longer blocks)
constexpr int LA_TPT = 4;    // tiles per thread (a block of at most 2,048 tiles)
constexpr int LA_GR = 4;     // rounds of 64 tiles whose scores are loaded at once
constexpr int L_LA_HOT = L_LA_STAGE;  // the tiles to read [2048]
static_assert(FU_THREADS * LA_TPT * 32 == 65536 && 4 * FU_THREADS * LA_TPT <= LA_SCAN_MAX * 4,
              "a block of at most 2,048 tiles, their list inside the scores' place");

// The split's queries (loaded before the selection, so that their load overlaps it).
template <int HPW>
__device__ __forceinline__ void la_queries(const FusedArgs& a, int b, int j, u32x4 (&qv)[FuAtt<HPW>::QPT]) {
  const int tid = threadIdx.x, hg = j % a.HG;
  // (unconditional: a workgroup past the last split loads its head group's queries and never uses them)
  const u32x4* qsrc = reinterpret_cast<const u32x4*>(a.q + ((size_t)b * a.H + HPW * hg) * FU_DQK);
#pragma unroll
  for (int i = 0; i < FuAtt<HPW>::QPT; ++i) qv[i] = qsrc[min(tid + FU_THREADS * i, HPW * FU_DQK / 8 - 1)];
}

// fu_attend_prep's token form in two steps, the split's positions taken from pos_l (the output order) instead of idx:
// la_slot, thread t's slot of the split's output t (0 past the split), then la_stage, the slot list and the unit's
// queries into LDS
template <int HPW>
__device__ __forceinline__ int la_slot(const FusedArgs& a, const int* pos_l, int b, int s, int cnt_row) {
  const int tid = threadIdx.x;
  const bool active = s < a.S;
  const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
  const int o = o0 + tid;
  int sl = 0;
  if (tid < FuAtt<HPW>::SPLIT && o < o1 && o < max(cnt_row, 1)) {  // the empty row lists output 0 (position 0)
    const int p = max(pos_l[tid], 0), pi = p / a.page_size;
    const int pg = a.table[(size_t)b * a.max_pages + min(pi, a.max_pages - 1)];
    sl = safe_page(pg, a.num_pages) * a.page_size + (p - pi * a.page_size);
  }
  return (unsigned)sl < (unsigned)a.num_slots ? sl : 0;
}

// The unit's queries into LDS at qs, [HPW][AQROW] bf16.
template <int HPW>
__device__ __forceinline__ void la_put_queries(uint16_t* qs, const u32x4 (&qv)[FuAtt<HPW>::QPT]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < FuAtt<HPW>::QPT; ++i) {
    const int pc = tid + FU_THREADS * i;
    if (pc < HPW * FU_DQK / 8)
      *reinterpret_cast<u32x4*>(qs + (pc / (FU_DQK / 8)) * FuAtt<HPW>::AQROW + 8 * (pc % (FU_DQK / 8))) = qv[i];
  }
}

// A second unit's queries, staged while the first unit attends: past the 32-head attention's LDS.
constexpr int L_LA_Q2 = FuAtt<32>::L_QST + 2 * 32 * FU_AQROW;
static_assert(L_LA_Q2 + 2 * 32 * FU_AQROW <= FU_LDS && FuAtt<32>::L_QST >= FuAtt<32>::L_END,
              "the second unit's queries clear of the first's attention");

template <int HPW>
__device__ __forceinline__ int la_stage(const FusedArgs& a, uint8_t* lds, int sl, int s, int cnt_row,
                                        const u32x4 (&qv)[FuAtt<HPW>::QPT], float* live_bias) {
  using AT = FuAtt<HPW>;
  int* slot_l = reinterpret_cast<int*>(lds + AT::L_P);
  const int tid = threadIdx.x;
  const bool active = s < a.S;
  const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
  if (active) la_put_queries<HPW>(reinterpret_cast<uint16_t*>(lds + AT::L_QST), qv);
  if (tid < AT::CAP) slot_l[tid] = sl;  // padding rows read slot 0 (the slot list lies before the positions)
  int n_slots = max(min(o1, cnt_row) - o0, 0);
  *live_bias = 0.0f;
  if (active && cnt_row == 0 && s == 0) {
    n_slots = 1;
    *live_bias = NEG_INF;
  }
  __syncthreads();  // the slot list and the queries
  return n_slots;
}

// Stage 2 and the split's positions (stage 3) over the row's 32 lists, their counts in LDS (lcnt). The T search of
// the one-exchange selection: the next 12 and 8 bits from the keys in c0 (c0 = -1: T = 0, every listed key taken),
// each list's keys above and at T, the ties taken (room: the lowest positions, list order then position order) and
// each list's first output index; then every selected key's output index, the split's [o0, o1) into pos_l.
// la_select_regs: every list of at most LA_LCAP entries, held in registers (thread (w, q): list w's entries
// 16 q .. 16 q + 15, one round of loads); la_select_loop: any lists, passed from the L2 (a list at a time).
constexpr int LA_LPT = 16, LA_LCAP = 16 * LA_LPT;
// (the second level's counts in bins1 and their coarse bins in co1, by every wave alike)
__device__ __forceinline__ void la_t_search(const FusedArgs& a, uint8_t* lds, int c0, int above0, uint32_t* T,
                                            int* room) {
  const int* bins1 = reinterpret_cast<const int*>(lds + L_BINS);
  const int* co1 = reinterpret_cast<const int*>(lds + L_CO1);
  int c1, above1;
  int need = a.keep - above0;
  fu_wave_find(bins1, co1, need, &c1, &above1);
  need -= above1;
  *T = ((uint32_t)c0 << 20) | ((uint32_t)c1 << 8);
  *room = need;  // (need >= bins1[c1]: every key of bin c1 is taken, T its lowest key with all its ties)
}

// A key of bin c0 into the second level's counts.
__device__ __forceinline__ void la_add1(uint8_t* lds, uint32_t k) {
  atomicAdd(reinterpret_cast<int*>(lds + L_BINS) + ((k >> 8) & 4095u), 1);
  atomicAdd(reinterpret_cast<int*>(lds + L_CO1) + ((k >> 14) & 63u), 1);
}

__device__ __forceinline__ void la_select_regs(const FusedArgs& a, uint8_t* lds, const uint32_t* lst_b,
                                               size_t lrow_words, int c0, int above0, int o0, int o1, int* pos_l) {
  int* bins1 = reinterpret_cast<int*>(lds + L_BINS);
  int* bins2 = reinterpret_cast<int*>(lds + L_BINS2);
  int* lcnt = reinterpret_cast<int*>(lds + L_LA);
  int *lgt = lcnt + FU_NW, *leq = lcnt + 2 * FU_NW, *ltake = lcnt + 3 * FU_NW, *loff = lcnt + 4 * FU_NW;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int w = tid >> 4, q = tid & 15;
  const int nw = lcnt[w] - LA_LPT * q;  // this thread's entries: those below nw
  const uint32_t* src = lst_b + (size_t)w * lrow_words + LA_HDR + 2 * LA_LPT * q;
  u32x4 ev[LA_LPT / 2];
#pragma unroll
  for (int i = 0; i < LA_LPT / 2; ++i)
    ev[i] = i * 2 < nw ? reinterpret_cast<const u32x4*>(src)[i] : u32x4{0u, 0u, 0u, 0u};
  uint32_t key[LA_LPT], pos[LA_LPT];
#pragma unroll
  for (int i = 0; i < LA_LPT; ++i) {
    key[i] = i < nw ? ev[i / 2][2 * (i & 1)] : 0u;
    pos[i] = ev[i / 2][2 * (i & 1) + 1];
  }
  uint32_t T = 0u;
  int room = 0;
  if (c0 >= 0) {
#pragma unroll
    for (int i = 0; i < LA_LPT; ++i)
      if (key[i] && (int)(key[i] >> 20) == c0) la_add1(lds, key[i]);
    __syncthreads();
    la_t_search(a, lds, c0, above0, &T, &room);
    const int c1 = (int)((T >> 8) & 4095u);
    if (room < bins1[c1]) {
      const uint32_t hi24 = T >> 8;
#pragma unroll
      for (int i = 0; i < LA_LPT; ++i)
        if (key[i] && (key[i] >> 8) == hi24) atomicAdd(&bins2[key[i] & 255u], 1);
      __syncthreads();
      int c2, above2;
      fu_wave_find256(bins2, room, &c2, &above2);
      T |= (uint32_t)c2;
      room = max(room - above2, 0);
    }
  }
  // per list: its keys above and at T (packed counts, summed over its 16 threads in list order)
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < LA_LPT; ++i) mine += (key[i] > T ? 1u : 0u) + (key[i] == T && key[i] ? 0x10000u : 0u);
  const uint32_t incl = (uint32_t)row_incl_scan((int)mine);
  if (q == 15) {
    lgt[w] = (int)(incl & 0xFFFFu);
    leq[w] = (int)(incl >> 16);
  }
  __syncthreads();
  const int ww = lane & (FU_NW - 1);
  const int eqw = lane < FU_NW ? leq[ww] : 0;
  const int tbw = wave_incl_scan(eqw) - eqw;
  const int takew = lane < FU_NW ? min(max(room - tbw, 0), eqw) : 0;
  const int selw = lane < FU_NW ? lgt[ww] + takew : 0;
  const int offw = wave_incl_scan(selw) - selw;
  const int off_l = __shfl(offw, w, WAVE), take_l = __shfl(takew, w, WAVE);
  // the selected entries meeting the split: each entry's output index from its list's first, the list's keys above
  // T before it and its ties taken before it (as the one-launch layer's one-exchange selection)
  int gtb = (int)((incl - mine) & 0xFFFFu), eqb = (int)((incl - mine) >> 16);
  const int first = off_l + gtb + min(eqb, take_l);
  const int nsel = (int)(mine & 0xFFFFu) + min(max(take_l - eqb, 0), (int)(mine >> 16));
  if (nsel > 0 && first < o1 && first + nsel > o0) {
    const int nties = (int)(mine >> 16);
    if (nties == 0 || eqb >= take_l || eqb + nties <= take_l) {
      const uint32_t thr = nties > 0 && eqb < take_l ? T : T + 1u;
      int r = first - o0;
#pragma unroll
      for (int i = 0; i < LA_LPT; ++i) {
        const bool sl = key[i] >= thr;
        if (sl && (unsigned)r < (unsigned)(o1 - o0)) pos_l[r] = (int)pos[i];
        r += sl;
      }
    } else {
#pragma unroll
      for (int i = 0; i < LA_LPT; ++i) {
        const bool above = key[i] > T, tie = key[i] == T && key[i];
        const int o = off_l + gtb + min(eqb, take_l) - o0;
        if ((above || (tie && eqb < take_l)) && (unsigned)o < (unsigned)(o1 - o0)) pos_l[o] = (int)pos[i];
        gtb += above;
        eqb += tie;
      }
    }
  }
  (void)ltake, (void)loff;
}

__device__ __forceinline__ void la_select_loop(const FusedArgs& a, uint8_t* lds, const uint32_t* lst_b,
                                               size_t lrow_words, int c0, int above0, int o0, int o1, int* pos_l) {
  int* scr = reinterpret_cast<int*>(lds + L_MISC);
  int* bins1 = reinterpret_cast<int*>(lds + L_BINS);
  int* bins2 = reinterpret_cast<int*>(lds + L_BINS2);
  int* lcnt = reinterpret_cast<int*>(lds + L_LA);
  int *lgt = lcnt + FU_NW, *leq = lcnt + 2 * FU_NW, *ltake = lcnt + 3 * FU_NW, *loff = lcnt + 4 * FU_NW;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  uint32_t T = 0u;
  int room = 0;
  if (c0 >= 0) {
    for (int w = 0; w < FU_NW; ++w) {
      const uint2* e = reinterpret_cast<const uint2*>(lst_b + (size_t)w * lrow_words + LA_HDR);
      for (int i = tid; i < lcnt[w]; i += FU_THREADS) {
        const uint32_t k = e[i].x;
        if ((int)(k >> 20) == c0) la_add1(lds, k);
      }
    }
    __syncthreads();
    la_t_search(a, lds, c0, above0, &T, &room);
    const int c1 = (int)((T >> 8) & 4095u);
    if (room < bins1[c1]) {
      const uint32_t hi24 = T >> 8;
      for (int w = 0; w < FU_NW; ++w) {
        const uint2* e = reinterpret_cast<const uint2*>(lst_b + (size_t)w * lrow_words + LA_HDR);
        for (int i = tid; i < lcnt[w]; i += FU_THREADS) {
          const uint32_t k = e[i].x;
          if ((k >> 8) == hi24) atomicAdd(&bins2[k & 255u], 1);
        }
      }
      __syncthreads();
      int c2, above2;
      fu_wave_find256(bins2, room, &c2, &above2);
      T |= (uint32_t)c2;
      room = max(room - above2, 0);
    }
  }
  // per list: its keys above T and at T
  for (int w = 0; w < FU_NW; ++w) {
    const uint2* e = reinterpret_cast<const uint2*>(lst_b + (size_t)w * lrow_words + LA_HDR);
    int g = 0, q = 0;
    for (int i = tid; i < lcnt[w]; i += FU_THREADS) {
      const uint32_t k = e[i].x;
      g += k > T;
      q += k == T;
    }
    if (g) atomicAdd(&lgt[w], g);
    if (q) atomicAdd(&leq[w], q);
  }
  __syncthreads();
  if (tid < WAVE) {  // wave 0: the ties taken (while fewer than room come before) and each list's first output
    const int eqw = lane < FU_NW ? leq[lane] : 0;
    const int tbw = wave_incl_scan(eqw) - eqw;
    const int takew = lane < FU_NW ? min(max(room - tbw, 0), eqw) : 0;
    const int selw = lane < FU_NW ? lgt[lane] + takew : 0;
    const int offw = wave_incl_scan(selw) - selw;
    if (lane < FU_NW) {
      ltake[lane] = takew;
      loff[lane] = offw;
    }
  }
  __syncthreads();
  // the split's positions, from the lists holding its outputs (a block prefix per pass of 512 entries)
  for (int w = 0; w < FU_NW; ++w) {  // workgroup-uniform
    const int ow = loff[w], sw = lgt[w] + ltake[w], n = lcnt[w], take = ltake[w];
    if (sw == 0 || ow >= o1 || ow + sw <= o0) continue;
    const uint2* e = reinterpret_cast<const uint2*>(lst_b + (size_t)w * lrow_words + LA_HDR);
    int gtc = 0, eqc = 0;  // the list's keys above and at T in the passes before
    for (int c = 0; c < n; c += FU_THREADS) {
      const int i = c + tid;
      const uint2 en = i < n ? e[i] : make_uint2(0u, 0u);
      const bool ab = en.x > T, tie = en.x == T && en.x;
      uint32_t tot;
      const uint32_t before = fu_block_prefix((ab ? 1u : 0u) | (tie ? 0x10000u : 0u), scr, &tot);
      const int gb = gtc + (int)(before & 0xFFFFu), eb = eqc + (int)(before >> 16);
      const int o = ow + gb + min(eb, take);
      if ((ab || (tie && eb < take)) && o >= o0 && o < o1) pos_l[o - o0] = (int)en.y;
      gtc += (int)(tot & 0xFFFFu);
      eqc += (int)(tot >> 16);
      __syncthreads();  // scr is written again by the next pass's prefix
    }
  }
}

constexpr int LA_RPL = 4;  // rows an XCD a launch at most

template <int HPW>
__global__ __launch_bounds__(FU_THREADS, 1) void decode_long_attend_kernel(FusedArgs a, LongAttArgs la) {
  __shared__ __align__(16) uint8_t lds[FU_LDS];
  using AT = FuAtt<HPW>;
  const int x = blockIdx.x % FU_XCDS, j = blockIdx.x / FU_XCDS;
  const FuSync sync = fu_sync_begin(a.sync + x * WS_SYNC_WORDS, j);
  if (a.row0 + x >= a.B) return;  // an XCD without a row
  const int nr = min(la.rpl, (a.B - a.row0 - x + FU_XCDS - 1) / FU_XCDS);  // this XCD's rows
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  int* scr = reinterpret_cast<int*>(lds + L_MISC);
  int* bins1 = reinterpret_cast<int*>(lds + L_BINS);
  int* bins2 = reinterpret_cast<int*>(lds + L_BINS2);
  int* lcnt = reinterpret_cast<int*>(lds + L_LA);  // per list: its entries, above T, at T, ties taken, first output
  int *lgt = lcnt + FU_NW, *leq = lcnt + 2 * FU_NW;
  int* pos_l = reinterpret_cast<int*>(lds + AT::L_P) + AT::CAP + 8;  // the split's positions (P's region)
  const size_t lrow_words = LA_HDR + 2 * (size_t)la.bw;
  for (int r = 0; r < nr; ++r) {
    const int b = a.row0 + x + FU_XCDS * r;
    const int L = min(max(a.ctx_len[b], 0), a.stride);
    if (r) __syncthreads();  // the previous row's stage 1 is done with the LDS
    // stage 1: the block's keys at or above c0 (every visible key when c0 = -1) into its list, in position order
    uint32_t* lrow = la.lst + ((size_t)b * FU_NW + j) * lrow_words;
    uint2* lent = reinterpret_cast<uint2*>(lrow + LA_HDR);
    const float* srow = a.scores + (size_t)b * a.stride;
    int listed = 0;
    int c0 = 0, above0 = 0;
    // the row in 32 blocks of bwb positions (at most the launch's bw), positions [pb, pe) of this workgroup's; with the
    // tile maxima a multiple of 128, thread t holding those of tiles tb + 4 t .. tb + 4 t + 3 (tiles [tb, te) of 32);
    // over the scores a multiple of 8, thread t taking positions 8 t .. 8 t + 7 of each pass of 4,096
    const bool tiles = la.tmax != nullptr;  // (launch-uniform)
    const int bq = tiles ? 128 : LA_PASS;
    const int bwb = min((L + FU_NW * bq - 1) / (FU_NW * bq) * bq, la.bw);
    const int pb = j * bwb, pe = min(pb + bwb, L);
    const int tb = pb / 32, te = tiles ? min((pe + 31) / 32, la.ntile) : 0;  // (a row longer than max_len: not past)
    const int npass = tiles ? 0 : (bwb + FU_THREADS * LA_PASS - 1) / (FU_THREADS * LA_PASS);
    float tm[LA_TPT];
    if (tiles) {
      const int t0 = tb + LA_TPT * tid;
      const float4 m4 = t0 < te ? *reinterpret_cast<const float4*>(la.tmax + (size_t)b * la.ntile + t0)
                                : make_float4(NEG_INF, NEG_INF, NEG_INF, NEG_INF);
      tm[0] = m4.x, tm[1] = m4.y, tm[2] = m4.z, tm[3] = m4.w;
    } else {
      // the block's scores straight into LDS (pass k in slot k: lane l of wave v's 8 floats at 2048 v + 16 l and
      // 2048 v + 1024 + 16 l, read back by the same lane), one round of loads
      for (int k = 0; k < npass; ++k) {
        const int pt = pb + FU_THREADS * LA_PASS * k + LA_PASS * tid;
        uint8_t* dst = lds + L_LA_STAGE + (FU_THREADS * LA_PASS * 4) * k + 2048 * (tid / WAVE);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float* src = srow + (pt + 4 * h < pe ? pt + 4 * h : 0);  // (past the block: a score never used)
          __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst + 1024 * h), 16, 0, 0);
        }
      }
    }
    // the bin c0 of the row's keep-th largest key (the histogram's bins 8 tid .. 8 tid + 7)
    int hv[8];
    {
      const int4* h4 = reinterpret_cast<const int4*>(la.hist + (size_t)b * FU_HBINS) + 2 * tid;
      *reinterpret_cast<int4*>(hv) = h4[0];
      *reinterpret_cast<int4*>(hv + 4) = h4[1];
    }
    if (tid == 0) scr[8] = -1;
    __syncthreads();
    const int nvis = fu_find_bin<8>(hv, a.keep, scr, &c0, &above0);
    if (nvis <= a.keep) c0 = -1;  // every visible key is selected
    // the keys of N consecutive positions from p0 (v: their scores; live: whether they are the block's) that are at
    // or above c0 (0: not listed), and their count
    auto keys_of = [&](const float* v, int N, int p0, bool live, uint32_t* key) __attribute__((always_inline)) {
      uint32_t n = 0;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const float x2 = live && p0 + i < pe ? v[i] : NEG_INF;
        key[i] = order_key(x2) & (0u - (uint32_t)(x2 > VISIBLE));
        if (key[i] && (int)(key[i] >> 20) < c0) key[i] = 0u;  // below the boundary bin: not listed
        n += key[i] != 0u;
      }
      return n;
    };
    if (tiles) {
      // the block's tiles that can hold a key at or above c0, in tile order
      int* hot = reinterpret_cast<int*>(lds + L_LA_HOT);
      uint32_t nh = 0;
      bool ht[LA_TPT];
#pragma unroll
      for (int i = 0; i < LA_TPT; ++i) {
        const uint32_t mk = order_key(tm[i]);
        ht[i] = tb + LA_TPT * tid + i < te && tm[i] > VISIBLE && (int)(mk >> 20) >= c0;
        nh += ht[i];
      }
      uint32_t nhot;
      uint32_t at = fu_block_prefix(nh, scr, &nhot);
#pragma unroll
      for (int i = 0; i < LA_TPT; ++i)
        if (ht[i]) hot[at++] = tb + LA_TPT * tid + i;
      __syncthreads();  // the tile list (and scr, written again below)
      // their scores, LA_GR rounds of 64 tiles a round of loads (thread t: 4 scores of tile t / 8 of the round)
      for (int g0 = 0; g0 < (int)nhot; g0 += 64 * LA_GR) {  // workgroup-uniform
        float4 sv[LA_GR];
#pragma unroll
        for (int r = 0; r < LA_GR; ++r) {
          const int hi = g0 + 64 * r + (tid >> 3);
          const int p0 = 32 * (hi < (int)nhot ? hot[hi] : tb) + 4 * (tid & 7);
          sv[r] = p0 < a.stride ? *reinterpret_cast<const float4*>(srow + p0)
                                : make_float4(NEG_INF, NEG_INF, NEG_INF, NEG_INF);
        }
#pragma unroll
        for (int r = 0; r < LA_GR; ++r) {
          if (g0 + 64 * r >= (int)nhot) break;  // workgroup-uniform
          const int hi = g0 + 64 * r + (tid >> 3);
          const int p0 = 32 * (hi < (int)nhot ? hot[hi] : tb) + 4 * (tid & 7);
          const float v[4] = {sv[r].x, sv[r].y, sv[r].z, sv[r].w};
          uint32_t key[4], tot;
          const uint32_t mine = keys_of(v, 4, p0, hi < (int)nhot, key);
          uint32_t e = (uint32_t)listed + fu_block_prefix(mine, scr, &tot);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (key[i]) lent[e++] = make_uint2(key[i], (uint32_t)(p0 + i));
          listed += (int)tot;
          __syncthreads();  // scr is written again by the next round's prefix
        }
      }
    } else {
      __builtin_amdgcn_s_waitcnt(0);  // (the lane's own loads: no barrier)
      for (int k = 0; k < npass; ++k) {
        const int pt = pb + FU_THREADS * LA_PASS * k + LA_PASS * tid;
        const uint8_t* src = lds + L_LA_STAGE + (FU_THREADS * LA_PASS * 4) * k + 2048 * (tid / WAVE) + 16 * lane;
        const float4 f0 = *reinterpret_cast<const float4*>(src), f1 = *reinterpret_cast<const float4*>(src + 1024);
        const float v[LA_PASS] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        uint32_t key[LA_PASS], tot;
        const uint32_t mine = keys_of(v, LA_PASS, pt, true, key);
        uint32_t e = (uint32_t)listed + fu_block_prefix(mine, scr, &tot);
#pragma unroll
        for (int i = 0; i < LA_PASS; ++i)
          if (key[i]) lent[e++] = make_uint2(key[i], (uint32_t)(pt + i));
        listed += (int)tot;
        __syncthreads();  // scr is written again by the next pass's prefix
      }
    }
    // the list's count, and for stage 2 the row's boundary bin, the keys above it and its visible keys
    if (tid == 0) *reinterpret_cast<uint4*>(lrow) = uint4{(uint32_t)listed, (uint32_t)c0, (uint32_t)above0, (uint32_t)nvis};
  }
  fu_barrier(sync, 1);  // every block's list of the XCD's rows (and every workgroup past their histograms' reads)
  for (int r = 0; r < nr; ++r)
    if (tid < FU_HBINS / FU_NW / 4)  // the row's histogram back to zero, 1/32 by each workgroup
      reinterpret_cast<uint4*>(la.hist + (size_t)(a.row0 + x + FU_XCDS * r) * FU_HBINS + (FU_HBINS / FU_NW) * j)[tid] =
          uint4{0u, 0u, 0u, 0u};
  // stages 2-4 a row at a time, or two rows at once: with 32 heads a workgroup and an even number of head groups,
  // workgroups 0-15 take row r and 16-31 row r + 1, each its row's selection once and then the two head groups of one
  // split (units 2 u and 2 u + 1, u = j mod 16, of the row's 32; the second attends the rows the first gathered, its
  // queries staged past the row tile), where taking the rows in turn costs each workgroup two selections
  static_assert(FuAtt<32>::L_QST >= FuAtt<32>::L_P, "the 32-head queries past the row tile");
  for (int r = 0; r < nr;) {
    const bool paired = HPW == 32 && a.HG % 2 == 0 && r + 1 < nr;  // (launch-uniform)
    const int b = a.row0 + x + FU_XCDS * (paired ? r + j / (FU_NW / 2) : r);
    const int u0 = paired ? 2 * (j % (FU_NW / 2)) : j;  // the first unit (split u0 / HG, head group u0 mod HG)
    const int hg = u0 % a.HG, s = u0 / a.HG;
    const bool active = s < a.S;
    const int o0 = active ? s * a.sps : 0, o1 = active ? min(o0 + a.sps, a.keep) : 0;
    if (r) __syncthreads();  // the previous rows' attention is done with the LDS
    // stage 2: the lists' counts, then T and the ties to take (the split's queries loading meanwhile, issued after
    // the counts: the loads complete in order, so the counts' wait does not include the queries')
    const uint32_t* lst_b = la.lst + (size_t)b * FU_NW * lrow_words;
    const uint4 hdr = *reinterpret_cast<const uint4*>(lst_b + (size_t)j * lrow_words);  // this workgroup's own words
    const int lc = tid < FU_NW ? (int)lst_b[(size_t)tid * lrow_words] : 0;
    u32x4 qv[AT::QPT];
    la_queries<HPW>(a, b, u0, qv);
    const int c0 = (int)hdr.y, above0 = (int)hdr.z, nvis = (int)hdr.w;
    for (int i = tid; i < 4096; i += FU_THREADS) bins1[i] = 0;
    if (tid < 256) bins2[tid] = 0;
    if (tid < 64) reinterpret_cast<int*>(lds + L_CO1)[tid] = 0;
    if (tid < FU_NW) lgt[tid] = leq[tid] = 0;
    if (tid < AT::SPLIT) pos_l[tid] = 0;  // outputs past the count are 0
    if (tid == 0) scr[24] = scr[40] = -1;
    if (tid < FU_NW) lcnt[tid] = min(lc, la.bw);
    __syncthreads();
    const int cnt_row = min(nvis, a.keep);
    const int lmax = (int)wave_max_u32(lane < FU_NW ? (uint32_t)lcnt[lane] : 0u);
    if (lmax <= LA_LCAP) {
      la_select_regs(a, lds, lst_b, lrow_words, c0, above0, o0, o1, pos_l);
    } else {
      la_select_loop(a, lds, lst_b, lrow_words, c0, above0, o0, o1, pos_l);
    }
    if (u0 == 0 && tid == 0) a.cnt[b] = cnt_row;
    __syncthreads();  // the split's positions
    if (hg == 0 && tid < o1 - o0) a.idx[(size_t)b * a.keep + o0 + tid] = pos_l[tid];
    const int sl = la_slot<HPW>(a, pos_l, b, s, cnt_row);
    // paired: the second unit's queries load while the first unit's stage
    u32x4 qv1[AT::QPT];
    if (paired) la_queries<HPW>(a, b, u0 + 1, qv1);
    float live_bias;
    const int n_slots = la_stage<HPW>(a, lds, sl, s, cnt_row, qv, &live_bias);
    if (paired) la_put_queries<HPW>(reinterpret_cast<uint16_t*>(lds + L_LA_Q2), qv1);  // (read after a barrier)
    fu_attend<HPW>(a, lds, b, u0, n_slots, live_bias);
    if (paired) {
      __syncthreads();  // the first unit's attention is done with the LDS
      fu_attend<HPW>(a, lds, b, u0 + 1, n_slots, live_bias, false, L_LA_Q2);
    }
    r += paired ? 2 : 1;
  }
  fu_barrier(sync, 2);  // every split's output of the XCD's rows
  for (int r = 0; r < nr; ++r) fu_combine(a, lds, a.row0 + x + FU_XCDS * r, j);
  fu_exit(sync, 2);
}

// ---- host side ----

static size_t fu_up256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace of the fused layer past the zero region (histograms + barrier words; the fused layer uses only the barrier
// words): the per-workgroup bin lists and candidate blocks, the split outputs and their (max, sum).
struct FusedLayout {
  size_t hl, cand, lst, part, ml, end;
};

static FusedLayout fused_layout(size_t zero_bytes, int B, int H, int S) {
  FusedLayout l;
  l.hl = zero_bytes;
  l.cand = l.hl + fu_up256((size_t)B * FU_NW * FU_HROW * 4);
  l.lst = l.cand + fu_up256((size_t)B * FU_NW * FU_CROW * 4);
  l.part = l.lst + fu_up256((size_t)B * FU_NW * FU_LROW * 4);
  l.ml = l.part + fu_up256((size_t)B * S * H * FU_DV * 2);
  l.end = l.ml + fu_up256((size_t)B * S * H * sizeof(float2));
  return l;
}

// The attention's heads per workgroup: 32 when the splits of 128 slots hold keep, else 16 (splits of 256); 0: no
// fused layer for these head counts.
static int fused_hpw(int H, int keep) {
  if (H >= 32 && H % 32 == 0 && H / 32 <= FU_NW && (long)(FU_NW / (H / 32)) * FuAtt<32>::SPLIT >= keep) return 32;
  if (H >= 16 && H % 16 == 0 && H / 16 <= FU_NW && (long)(FU_NW / (H / 16)) * FuAtt<16>::SPLIT >= keep) return 16;
  return 0;
}

static int fused_splits(int H, int hpw) { return FU_NW / (H / hpw); }

// Whether the fused layer takes a step: a GPU of 8 XCDs x 32 CUs, rows of at most 32,768 tokens (score rows of a
// multiple of 4 floats), up to 64 indexer heads, query heads in 16s (at most 512), pages of a power-of-two size of at
// least 32 tokens, and a keep that the splits hold (128 slots each at 32 heads per workgroup, 256 at 16).
bool fused_layer_ok(int num_cu, int Hi, int H, int max_len, int keep, int page_size, int stride) {
  if (num_cu != FU_XCDS * FU_NW) return false;
  if (Hi < 1 || Hi > 64 || keep < 1 || !fused_hpw(H, keep)) return false;
  if (max_len < 1 || max_len > FU_MAXLEN || stride < 1 || stride % 4) return false;
  return page_size >= 32 && !(page_size & (page_size - 1));
}

size_t fused_layer_bytes(size_t zero_bytes, int B, int H, int keep) {
  const int hpw = keep >= 1 ? fused_hpw(H, keep) : 0;
  if (!hpw) return 0;
  return fused_layout(zero_bytes, B, H, fused_splits(H, hpw)).end;
}

// The separate attention launch (decode_attend_kernel): whether it takes the shape, and its workspace (the split
// outputs and their (max, sum)).
bool attend_xcd_ok(int num_cu, int H, int keep) { return num_cu == FU_XCDS * FU_NW && keep >= 1 && fused_hpw(H, keep); }

size_t attend_xcd_bytes(int B, int H, int keep) {
  const int hpw = keep >= 1 ? fused_hpw(H, keep) : 0;
  if (!hpw) return 0;
  const FusedLayout l = fused_layout(0, B, H, fused_splits(H, hpw));
  return l.end - l.part;
}

// The separate attention launch's arguments past the selection's (rows, idx, cnt, npool, positions, kp_shift): the
// split outputs in ws, the per-XCD barrier words in sync, splits of a multiple of 64 slots over `keep` slots a row.
static FusedArgs attend_args(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table, uint16_t* out,
                             float* lse, void* ws, int* sync, int B, int H, int max_pages, int page_size,
                             int num_pages, int keep, float scale, int hpw) {
  FusedArgs a{};
  const int S = fused_splits(H, hpw);
  const FusedLayout l = fused_layout(0, B, H, S);
  char* p = static_cast<char*>(ws) - l.part;
  a.q = q;
  a.kv = kv;
  a.kvs = kvs;
  a.table = table;
  a.out = out;
  a.lse = lse;
  a.sync = sync;
  a.part = reinterpret_cast<uint16_t*>(p + l.part);
  a.ml = reinterpret_cast<float2*>(p + l.ml);
  a.B = B;
  a.H = H;
  a.max_pages = max_pages;
  a.page_size = page_size;
  a.num_pages = num_pages;
  a.num_slots = num_pages * page_size;
  a.keep = keep;
  a.scale = scale;
  a.HG = H / hpw;
  a.S = S;
  int sps = (keep + S - 1) / S;
  a.sps = (sps + FU_CH - 1) / FU_CH * FU_CH;
  return a;
}

// One launch per 4 rows per XCD at most: a batch of 12 rows is one launch of 2 rows per XCD (or 1), not 8 + 4.
template <typename K>
static hipError_t attend_launches(FusedArgs a, K kernel, const int* rows, hipStream_t s) {
  const dim3 grid(FU_XCDS * FU_NW), block(FU_THREADS);
  constexpr int RPL_MAX = 4;
  for (int r0 = 0; r0 < a.B; r0 += FU_XCDS * RPL_MAX) {
    a.row0 = r0;
    const int left = a.B - r0, rpl = (left < FU_XCDS * RPL_MAX ? left : FU_XCDS * RPL_MAX) + FU_XCDS - 1;
    const hipError_t e = launch("decode_attend_kernel", kernel, grid, block, s, a, rows, rpl / FU_XCDS);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_decode_attend(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* rows,
                                const int* idx, const int* table, const int* cnt, uint16_t* out, float* lse, void* ws,
                                int* sync, int B, int H, int max_pages, int page_size, int num_pages, int keep,
                                float scale, hipStream_t s) {
  const int hpw = fused_hpw(H, keep);
  if (!hpw || (!rows && (!idx || !table))) return hipErrorInvalidValue;
  FusedArgs a = attend_args(q, kv, kvs, table, out, lse, ws, sync, B, H, max_pages, page_size, num_pages, keep, scale,
                            hpw);
  a.idx = const_cast<int*>(idx);
  a.cnt = const_cast<int*>(cnt);
  return hpw == 32 ? attend_launches(a, decode_attend_kernel<32>, rows, s)
                   : attend_launches(a, decode_attend_kernel<16>, rows, s);
}

// The long rows' selection, attention and combine in one launch (decode_long_attend_kernel): rows past 32,768
// tokens (at most LA_MAXLEN), the attention's head shapes, score rows of a multiple of 4 floats.
static int la_block(long max_len) {
  const long per = (max_len + FU_NW - 1) / FU_NW, q = 4096;  // (a multiple of 4 tiles a thread)
  return (int)((per + q - 1) / q * q);
}

// The tiles per row of the tile maxima (a multiple of 4: each thread reads 4 with one 16-byte load).
static int la_ntile(long max_len) { return (int)((max_len + 127) / 128 * 4); }

// Whether stage 1 reads the tile maxima (blocks longer than one round of score loads).
bool long_attend_tiles(long max_len) { return la_block(max_len) > LA_SCAN_MAX; }

bool long_attend_ok(int num_cu, int H, int keep, long max_len, int stride) {
  return num_cu == FU_XCDS * FU_NW && keep >= 1 && fused_hpw(H, keep) && max_len > FU_MAXLEN &&
         max_len <= LA_MAXLEN && stride >= max_len && stride % 4 == 0;
}

// Its workspace past the top-k's: the split outputs and their (max, sum), the blocks' lists, then the rows' tile
// maxima (written by the long-row indexer before the launch).
size_t long_attend_bytes(int B, int H, int keep, long max_len) {
  if (keep < 1 || !fused_hpw(H, keep) || max_len <= FU_MAXLEN || max_len > LA_MAXLEN) return 0;
  return fu_up256(attend_xcd_bytes(B, H, keep)) +
         fu_up256((size_t)B * FU_NW * (LA_HDR + 2 * (size_t)la_block(max_len)) * 4) +
         fu_up256((size_t)B * la_ntile(max_len) * 4);
}

// The tile maxima's place in that workspace and their tiles per row (the long-row indexer's bm and nb, tiles of 32).
float* long_attend_tmax(void* ws, int B, int H, int keep, long max_len) {
  return reinterpret_cast<float*>(static_cast<char*>(ws) + fu_up256(attend_xcd_bytes(B, H, keep)) +
                                  fu_up256((size_t)B * FU_NW * (LA_HDR + 2 * (size_t)la_block(max_len)) * 4));
}
int long_attend_ntile(long max_len) { return la_ntile(max_len); }

hipError_t launch_decode_long_attend(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                                     const int* ctx_len, const float* scores, int stride, int* hist, int* idx,
                                     int* cnt, uint16_t* out, float* lse, void* ws, int* sync, int B, int H,
                                     int max_pages, int page_size, int num_pages, int keep, float scale, long max_len,
                                     hipStream_t s) {
  const int hpw = fused_hpw(H, keep);
  if (!hpw || max_len <= FU_MAXLEN || max_len > LA_MAXLEN || stride % 4) return hipErrorInvalidValue;
  FusedArgs a = attend_args(q, kv, kvs, table, out, lse, ws, sync, B, H, max_pages, page_size, num_pages, keep, scale,
                            hpw);
  a.scores = const_cast<float*>(scores);
  a.stride = stride;
  a.ctx_len = ctx_len;
  a.idx = idx;
  a.cnt = cnt;
  LongAttArgs la;
  la.hist = hist;
  la.bw = la_block(max_len);
  la.ntile = la_ntile(max_len);
  la.lst = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + fu_up256(attend_xcd_bytes(B, H, keep)));
  la.tmax = long_attend_tiles(max_len) ? long_attend_tmax(ws, B, H, keep, max_len) : nullptr;
  const dim3 grid(FU_XCDS * FU_NW), block(FU_THREADS);
  static_assert(2 <= (int)(FU_SPAN / FU_NW), "a launch's barriers within its span");
  for (int r0 = 0; r0 < B; r0 += FU_XCDS * LA_RPL) {
    a.row0 = r0;
    const int left = B - r0;
    la.rpl = ((left < FU_XCDS * LA_RPL ? left : FU_XCDS * LA_RPL) + FU_XCDS - 1) / FU_XCDS;
    const hipError_t e = hpw == 32 ? launch("decode_long_attend_kernel", decode_long_attend_kernel<32>, grid, block,
                                            s, a, la)
                                   : launch("decode_long_attend_kernel", decode_long_attend_kernel<16>, grid, block,
                                            s, a, la);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The pooled form: 512-wide rows, 32 heads per workgroup (splits of 128 token slots, the split holding a row's last
// selected token taking its tail too).
bool attend_xcd_pooled_ok(int num_cu, int H, int Dqk, int keep_tokens) {
  return num_cu == FU_XCDS * FU_NW && Dqk == 512 && keep_tokens >= 1 && fused_hpw(H, keep_tokens) == 32;
}

hipError_t launch_decode_attend_pooled(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* pools,
                                       const int* cnt, const int* npool, const int* positions, const int* table,
                                       uint16_t* out, float* lse, void* ws, int* sync, int B, int H, int max_pages,
                                       int page_size, int num_pages, int keep_pools, int kp_shift, float scale,
                                       hipStream_t s) {
  const int keep = keep_pools << kp_shift;  // token slots
  if (kp_shift < 1 || !pools || !cnt || !npool || !positions || !table || fused_hpw(H, keep) != 32)
    return hipErrorInvalidValue;
  FusedArgs a = attend_args(q, kv, kvs, table, out, lse, ws, sync, B, H, max_pages, page_size, num_pages, keep, scale,
                            32);
  a.idx = const_cast<int*>(pools);
  a.cnt = const_cast<int*>(cnt);
  a.npool = npool;
  a.positions = positions;
  a.kp_shift = kp_shift;
  return attend_launches(a, decode_attend_kernel<32, 512, true>, nullptr, s);
}

hipError_t launch_decode_fused(const uint16_t* q_idx, const float* w, const uint8_t* k, const float* ks,
                               const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                               const int* ctx_len, float* scores, int* idx, int* cnt, uint16_t* out, float* lse,
                               void* ws, size_t zero_bytes, int B, int Hi, int H, int max_pages, int page_size,
                               int num_pages, int stride, int keep, float scale, hipStream_t s) {
  FusedArgs a;
  const int hpw = fused_hpw(H, keep);
  if (!hpw) return hipErrorInvalidValue;
  const int S = fused_splits(H, hpw);
  const FusedLayout l = fused_layout(zero_bytes, B, H, S);
  char* p = static_cast<char*>(ws);
  a.q_idx = q_idx;
  a.w = w;
  a.k = k;
  a.ks = ks;
  a.q = q;
  a.kv = kv;
  a.kvs = kvs;
  a.table = table;
  a.ctx_len = ctx_len;
  a.scores = scores;
  a.idx = idx;
  a.cnt = cnt;
  a.out = out;
  a.lse = lse;
  a.hl = reinterpret_cast<uint32_t*>(p + l.hl);
  a.sync = reinterpret_cast<int*>(p);  // the workspace's first bytes
  a.cand = reinterpret_cast<uint32_t*>(p + l.cand);
  a.lst = reinterpret_cast<uint32_t*>(p + l.lst);
  a.part = reinterpret_cast<uint16_t*>(p + l.part);
  a.ml = reinterpret_cast<float2*>(p + l.ml);
  a.B = B;
  a.Hi = Hi;
  a.H = H;
  a.max_pages = max_pages;
  a.page_size = page_size;
  a.page_shift = __builtin_ctz((unsigned)page_size);
  a.num_pages = num_pages;
  a.num_slots = num_pages * page_size;
  a.stride = stride;
  a.keep = keep;
  a.scale = scale;
  a.HG = H / hpw;
  a.S = S;
  int sps = (keep + S - 1) / S;
  a.sps = (sps + FU_CH - 1) / FU_CH * FU_CH;
  const dim3 grid(FU_XCDS * FU_NW), block(FU_THREADS);
  for (int r0 = 0; r0 < B; r0 += FU_XCDS) {
    a.row0 = r0;
    const hipError_t e =
        Hi <= 32 ? (hpw == 32 ? launch("decode_fused_kernel", decode_fused_kernel<1, 32>, grid, block, s, a)
                              : launch("decode_fused_kernel", decode_fused_kernel<1, 16>, grid, block, s, a))
                 : (hpw == 32 ? launch("decode_fused_kernel", decode_fused_kernel<2, 32>, grid, block, s, a)
                              : launch("decode_fused_kernel", decode_fused_kernel<2, 16>, grid, block, s, a));
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}


// The pooled one-launch layer: whether it takes a step (a GPU of 8 XCDs x 32 CUs, 512-wide latent rows, at most 32
// indexer heads, rows of at most 8,192 pools, pages of a power-of-two number of at least 16 pools, and a keep whose
// token slots the 32-head splits of 128 hold), and its workspace past the zero region: the key lists, the split
// outputs and their (max, sum).
bool fused_pooled_ok(int num_cu, int Hi, int H, int Dqk, int stride, int kp, int page_size, int keep_pools) {
  if (num_cu != FU_XCDS * FU_NW || Dqk != 512 || Hi < 1 || Hi > 32 || keep_pools < 1) return false;
  if (kp < 2 || kp > 8 || (kp & (kp - 1)) || page_size % kp) return false;
  const int ppp = page_size / kp;
  if (ppp < 16 || (ppp & (ppp - 1)) || stride < 1 || stride > FU_POOL_MAXLEN || stride % 4) return false;
  return fused_hpw(H, keep_pools * kp) == 32 && FuAtt<32>::SPLIT % kp == 0;
}

// Whether the one-launch pooled layer also takes the step's pool-key write (kpool FU_STEP_KP).
bool fused_step_ok(int kp) { return kp == FU_STEP_KP; }

size_t fused_pooled_bytes(size_t zero_bytes, int B, int H) {
  if (H < 32 || H % 32) return 0;
  const int S = fused_splits(H, 32);
  size_t off = zero_bytes;
  off += fu_up256((size_t)B * FU_NW * FuForm<true>::LROW * 4);
  off += fu_up256((size_t)B * S * H * FU_DV * 2);
  off += fu_up256((size_t)B * S * H * sizeof(float2));
  return off;
}

hipError_t launch_decode_fused_pooled(const uint16_t* q_idx, const float* w, const uint16_t* pool_key,
                                      const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                                      const int* npool, const int* positions, float* scores, int* pools, int* cnt,
                                      uint16_t* out, float* lse, void* ws, size_t zero_bytes, int B, int Hi, int H,
                                      int max_pages, int page_size, int num_pages, int kp, int keep_pools,
                                      float scale, const PoolKeyWrite* pkw, hipStream_t s) {
  FusedArgs a{};
  const int S = fused_splits(H, 32);
  char* p = static_cast<char*>(ws);
  const size_t lst = zero_bytes;
  const size_t part = lst + fu_up256((size_t)B * FU_NW * FuForm<true>::LROW * 4);
  const size_t ml = part + fu_up256((size_t)B * S * H * FU_DV * 2);
  const int ppp = page_size / kp;
  a.q_idx = q_idx;
  a.w = w;
  a.k = reinterpret_cast<const uint8_t*>(pool_key);
  a.ks = nullptr;
  a.q = q;
  a.kv = kv;
  a.kvs = kvs;
  a.table = table;
  a.ctx_len = npool;
  a.scores = scores;
  a.idx = pools;
  a.cnt = cnt;
  a.out = out;
  a.lse = lse;
  a.hl = nullptr;  // (no bin lists: the pooled form's key lists hold every key)
  a.sync = reinterpret_cast<int*>(p);  // the workspace's first bytes
  a.cand = nullptr;
  a.lst = reinterpret_cast<uint32_t*>(p + lst);
  a.part = reinterpret_cast<uint16_t*>(p + part);
  a.ml = reinterpret_cast<float2*>(p + ml);
  a.B = B;
  a.Hi = Hi;
  a.H = H;
  a.max_pages = max_pages;
  a.page_size = page_size;
  a.page_shift = __builtin_ctz((unsigned)page_size);
  a.num_pages = num_pages;
  a.num_slots = num_pages * page_size;
  a.stride = max_pages * ppp;
  a.keep = keep_pools;
  a.scale = scale;
  a.HG = H / 32;
  a.S = S;
  a.sps = FuAtt<32>::SPLIT / kp;  // pools per split (their token slots fill one split)
  a.npool = npool;
  a.positions = positions;
  a.kp_shift = __builtin_ctz((unsigned)kp);
  a.ppp_shift = __builtin_ctz((unsigned)ppp);
  if (pkw) {
    a.pk_rows = pkw->rows;
    a.pk_scale = pkw->rows_scale;
    a.pk_ape = pkw->ape;
    a.slot_mapping = pkw->slot_mapping;
    a.pk_width = pkw->rows_width;
    a.pk_fp8 = pkw->rows_fp8;
  }
  if (pkw && kp != FU_STEP_KP) return hipErrorInvalidValue;  // (fused_step_ok)
  const dim3 grid(FU_XCDS * FU_NW), block(FU_THREADS);
  for (int r0 = 0; r0 < B; r0 += FU_XCDS) {
    a.row0 = r0;
    const hipError_t e =
        pkw ? launch("decode_pooled_fused_kernel", decode_pooled_fused_kernel<32, true>, grid, block, s, a)
            : launch("decode_pooled_fused_kernel", decode_pooled_fused_kernel<32, false>, grid, block, s, a);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dsa
