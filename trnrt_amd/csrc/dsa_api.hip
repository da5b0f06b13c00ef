// C ABI entry points of libdsa_gfx950.so (declared in include/dsa_gfx950.h): host-side argument checks, launch
// shapes, and the launches on the caller's stream (the prefill selection also on the library's second stream, joined
// back to the caller's by events). Nothing here allocates device memory or synchronises the host.
#include "../../include/dsa_gfx950.h"

#include <mutex>

#include "dsa_common.h"

namespace dsa {
hipError_t launch_indexer_decode(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                 const int* table, const int* ctx_len, const float* cand, float* scores, int* hist,
                                 int B, int Hi, int max_pages, int page_size, int num_pages, int stride, int num_cu,
                                 hipStream_t stream);
hipError_t launch_indexer_prefill(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                  const int* npool, float* scores, int N, int Hi, int P, int stride, float scale,
                                  float* bm, int sub_log2, int nb, hipStream_t s);
hipError_t launch_indexer_prefill_fp8(const uint8_t* q8, const float* qs, const float* w, const uint8_t* k,
                                      const float* ks, const int* npool, float* scores, int N, int Hi, int P,
                                      int stride, float scale, float* bm, int sub_log2, int nb, hipStream_t s);
hipError_t launch_indexer_prefill_bf16k(const uint16_t* q, const float* w, const uint16_t* k, const int* npool,
                                        float* scores, int N, int Hi, int P, int stride, float scale, float* bm,
                                        int sub_log2, int nb, hipStream_t s);
int topk_two_level_sub(long n, int keep);
float* topk_bm_buffer(void* ws, int B);
hipError_t launch_prefill_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                               int n, int keep, bool bm_ready, int64_t* pools, int64_t* cnt64, float* vals,
                               hipStream_t s);
int prefill_tile_plan(long n, int stride, int keep);
hipError_t launch_prefill_tile_topk(const float* scores, int stride, const int* len, long n, int keep,
                                    const float* bm, int* bidx, int* bcnt, int64_t* pools, int64_t* cnt64,
                                    float* vals, int T, hipStream_t s);
bool cache_write_width_ok(int W);
hipError_t launch_cache_write(const void* x, int x_fp32, const int64_t* slots, uint8_t* cache, float* cscale,
                              int n_rows, int W, long num_slots, int scaled, float fp8_max, hipStream_t s);
hipError_t launch_pool_slots(const int* pools, const int* cnt, const int* npool, const int* positions,
                             const int* table, int table_shared, int* rows, float* bias, int N, int keep, int n_slots,
                             int table_pages, int page_size, int kp, hipStream_t s);
hipError_t launch_indexer_decode_bf16(const uint16_t* q, const float* w, const uint16_t* k, const int* table,
                                      const int* ctx_len, const float* cand, float* scores, int* hist, int B, int Hi,
                                      int max_pages, int page_size, int num_pages, int stride, hipStream_t s);
hipError_t launch_pool_keys(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                            const int* positions, const int* table, int table_shared, int table_pages,
                            const int64_t* slot_mapping, uint16_t* pool_key, int T, int kp, int page_size,
                            long num_slots, hipStream_t s);
hipError_t launch_topk(const float* scores, const int* len, int* idx, int* cnt, void* ws, int B, int stride,
                       int max_len, int keep, int vis_only, bool hist_ready, const int* table, int max_pages,
                       int page_size, int num_pages, int* rows_out, hipStream_t s, bool bm_ready = false);
hipError_t launch_indexer_decode_long(const uint16_t* q, const float* w, const uint8_t* k, const float* ks,
                                      const int* table, const int* ctx_len, float* scores, float* bm, int sub_log2,
                                      int nb, int* hist, int B, int Hi, int max_pages, int page_size, int num_pages,
                                      int stride, int num_cu, hipStream_t s);
bool topk_long_rows(int B, long n);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s);
hipError_t launch_topk_mask(const int* idx, const int* cnt, const float* scores, float* mask, int B, int keep, int P,
                            int kp, int tail, hipStream_t s);
size_t topk_workspace_bytes(int B, int max_len, int keep);
size_t topk_hist_bytes(int B);
size_t topk_zero_bytes(int B);
bool fused_layer_ok(int num_cu, int Hi, int H, int max_len, int keep, int page_size, int stride);
size_t fused_layer_bytes(size_t zero_bytes, int B, int H, int keep);
bool attend_xcd_ok(int num_cu, int H, int keep);
size_t attend_xcd_bytes(int B, int H, int keep);
hipError_t launch_decode_attend(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* rows,
                                const int* idx, const int* table, const int* cnt, uint16_t* out, float* lse, void* ws,
                                int* sync, int B, int H, int max_pages, int page_size, int num_pages, int keep,
                                float scale, hipStream_t s);
bool long_attend_ok(int num_cu, int H, int keep, long max_len, int stride);
size_t long_attend_bytes(int B, int H, int keep, long max_len);
float* long_attend_tmax(void* ws, int B, int H, int keep, long max_len);
int long_attend_ntile(long max_len);
bool long_attend_tiles(long max_len);
hipError_t launch_decode_long_attend(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                                     const int* ctx_len, const float* scores, int stride, int* hist, int* idx,
                                     int* cnt, uint16_t* out, float* lse, void* ws, int* sync, int B, int H,
                                     int max_pages, int page_size, int num_pages, int keep, float scale, long max_len,
                                     hipStream_t s);
bool attend_xcd_pooled_ok(int num_cu, int H, int Dqk, int keep_tokens);
hipError_t launch_decode_attend_pooled(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* pools,
                                       const int* cnt, const int* npool, const int* positions, const int* table,
                                       uint16_t* out, float* lse, void* ws, int* sync, int B, int H, int max_pages,
                                       int page_size, int num_pages, int keep_pools, int kp_shift, float scale,
                                       hipStream_t s);
hipError_t launch_decode_fused(const uint16_t* q_idx, const float* w, const uint8_t* k, const float* ks,
                               const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                               const int* ctx_len, float* scores, int* idx, int* cnt, uint16_t* out, float* lse,
                               void* ws, size_t zero_bytes, int B, int Hi, int H, int max_pages, int page_size,
                               int num_pages, int stride, int keep, float scale, hipStream_t s);
bool fused_pooled_ok(int num_cu, int Hi, int H, int Dqk, int stride, int kp, int page_size, int keep_pools);
size_t fused_pooled_bytes(size_t zero_bytes, int B, int H);
bool fused_step_ok(int kp);
hipError_t launch_decode_fused_pooled(const uint16_t* q_idx, const float* w, const uint16_t* pool_key,
                                      const uint16_t* q, const uint8_t* kv, const float* kvs, const int* table,
                                      const int* npool, const int* positions, float* scores, int* pools, int* cnt,
                                      uint16_t* out, float* lse, void* ws, size_t zero_bytes, int B, int Hi, int H,
                                      int max_pages, int page_size, int num_pages, int kp, int keep_pools,
                                      float scale, const PoolKeyWrite* pkw, hipStream_t s);
bool topk_supported(int max_len, int keep, int vis_only);
hipError_t launch_sparse_mla(const uint16_t* q, const uint8_t* kv, const float* kvs, const int* idx, const int* cnt,
                             const int* table, const int* rows, const float* bias, uint16_t* out, float* out_f32,
                             float* lse, void* ws, int B, int H, int Dqk, int keep, int max_pages, int page_size,
                             int num_pages, float scale, int splits, hipStream_t s, PoolForm pf = PoolForm{},
                             bool wide = false);
bool attention_wide_ok(int B, int H, int keep, bool has_bias, int num_cu);
hipError_t launch_token_rows(const int* idx, const int* cnt, const int* table, int* rows, float* bias, int B,
                             int keep, int max_pages, int page_size, int num_pages, hipStream_t s);
int attention_default_splits(int B, int H, int keep, int num_cu);
size_t attention_workspace_bytes(int B, int H, int splits);
hipError_t launch_compact_mask(const float* sel, int N, int M, int keep, int64_t* idx, int64_t* cnt, hipStream_t s);
hipError_t launch_compact_slots(const int* rows, const float* bias, int B, int NS, int kp, int pools, int* tok,
                                int* tcnt, hipStream_t s);
hipError_t launch_value_order(const int64_t* pools, const int64_t* cnt, const float* vals, int N, int keep,
                              int64_t* out_pools, float* out_vals, hipStream_t s);

thread_local KernelTimer* g_kernel_timer = nullptr;
}  // namespace dsa

// The scratch of dsa_decode_layer_noalloc: a file-scope device array of DSA_NOALLOC_SCRATCH_BYTES, one copy on each
// GPU the library runs on (held until the process ends). In host code `scratch` names a host-side stand-in, not a
// device address: the per-device address comes from hipGetSymbolAddress (noalloc_scratch below), and only that address
// reaches kernels and fills.
static __device__ __align__(256) uint8_t scratch[DSA_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local dsa::KernelTimer t_timer;

int num_cu() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

int status(hipError_t e) { return e == hipSuccess ? DSA_OK : DSA_ELAUNCH; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The layer's slot-id buffer [B, keep] int32 (between the top-k and the attention workspaces).
size_t layer_rows_bytes(int B, int keep) { return align256((size_t)B * keep * 4); }

int resolve_splits(int splits, int B, int H, int keep) {
  if (splits <= 0) splits = dsa::attention_default_splits(B, H, keep, num_cu());
  int max_splits = (keep + 63) / 64;  // whole 64-slot chunks per split, at most 32 splits (the combine's limit)
  max_splits = max_splits > 32 ? 32 : max_splits;
  return splits > max_splits ? max_splits : splits;
}

// The splits the launch really uses (whole 64-slot chunks per split).
int effective_splits(int splits, int keep) {
  int sps = (keep + splits - 1) / splits;
  sps = (sps + 63) / 64 * 64;
  return (keep + sps - 1) / sps;
}

// The prefill selection runs over tiles of T query rows: each tile's scores [T, score_stride] fp32, then its
// selection, so that nothing of the chunk's size x the context's is held at once (the reference's device form scores
// and selects per 128-query tile with two HBM score scratches, trnrt/kernels/dsa_long_pipe.py:15-25). By default a
// score tile is at most kPrefillTileBytes (equal tiles, whole groups of 4 rows: the indexer's workgroup).
constexpr size_t kPrefillTileBytes = 64ull << 20;

int prefill_tile_rows(int N, int stride, int tile_rows) {
  if (N <= 0) return 1;
  if (tile_rows > 0) return tile_rows < N ? tile_rows : N;
  long t = (long)(kPrefillTileBytes / ((size_t)stride * 4));
  if (t < 64) t = 64;
  if (t >= N) return N;
  const long tiles = (N + t - 1) / t;
  const long rows = ((N + tiles - 1) / tiles + 3) / 4 * 4;
  return (int)(rows < N ? rows : N);
}

// Workspace of the prefill selection, in order: the generic selection's workspace and its int32 outputs (plan < 0
// only; its zero region first), then `sets` score tiles (own scores only), and with plan > 0 `sets` each of the
// sub-block maxima tiles and of the first level's outputs. plan: dsa::prefill_tile_plan. Two sets when tiles
// alternate between two streams (plan >= 0 and more than one tile), else one.
struct PrefillLayout {
  int T, tiles, plan, sets;
  size_t gidx_off, gcnt_off, sc_off, sc_bytes, bm_off, bm_bytes, bidx_off, bidx_bytes, bcnt_off, bcnt_bytes, total;
};

PrefillLayout prefill_layout(int N, int P, int stride, int keep, int tile_rows, bool own_scores) {
  PrefillLayout L{};
  L.T = prefill_tile_rows(N, stride, tile_rows);
  L.tiles = N > 0 ? (N + L.T - 1) / L.T : 0;
  L.plan = dsa::prefill_tile_plan(P, stride, keep);
  L.sets = L.plan >= 0 && L.tiles > 1 ? 2 : 1;
  size_t off = 0;
  if (L.plan < 0) {
    off = align256(dsa::topk_workspace_bytes(L.T, P, keep));
    L.gidx_off = off;
    off += align256((size_t)L.T * keep * 4);
    L.gcnt_off = off;
    off += align256((size_t)L.T * 4);
  }
  L.sc_off = off;
  L.sc_bytes = own_scores ? align256((size_t)L.T * stride * 4) : 0;
  off += L.sets * L.sc_bytes;
  L.bm_off = off;
  if (L.plan > 0) {
    const long nb = (P + L.plan - 1) / L.plan;
    L.bm_bytes = align256((size_t)L.T * nb * 4);
    off += L.sets * L.bm_bytes;
    L.bidx_off = off;
    L.bidx_bytes = align256((size_t)L.T * keep * 4);
    off += L.sets * L.bidx_bytes;
    L.bcnt_off = off;
    L.bcnt_bytes = align256((size_t)L.T * 4);
    off += L.sets * L.bcnt_bytes;
  }
  L.total = off > 256 ? off : 256;
  return L;
}

constexpr int kMaxDevices = 64;

// The library's second stream on each device (default priority, not synchronising with the null stream), created on
// first use and kept until the process ends, with the two events that fork it from and join it to a caller's stream.
// One call at a time holds a device's set (the lock), so the events' records and waits of two calls never interleave.
std::mutex g_aux_mu;
hipStream_t g_aux_stream[kMaxDevices] = {};
hipEvent_t g_aux_events[kMaxDevices][2] = {};

struct AuxStream {
  bool ok = false;
  hipStream_t stream = nullptr;
  hipEvent_t start = nullptr, end = nullptr;
  std::unique_lock<std::mutex> lock;

  explicit AuxStream(bool want) {
    int dev = 0;
    if (!want || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
    lock = std::unique_lock<std::mutex>(g_aux_mu);
    if (!g_aux_stream[dev]) {
      hipStream_t s = nullptr;
      hipEvent_t ev[2] = {};
      bool made = hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess;
      for (int i = 0; i < 2 && made; ++i) made = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) == hipSuccess;
      if (!made) {
        for (hipEvent_t e : ev)
          if (e) (void)hipEventDestroy(e);
        if (s) (void)hipStreamDestroy(s);
        (void)hipGetLastError();  // the next launch's status must not report this failure
        lock.unlock();
        return;
      }
      g_aux_stream[dev] = s;
      g_aux_events[dev][0] = ev[0];
      g_aux_events[dev][1] = ev[1];
    }
    stream = g_aux_stream[dev];
    start = g_aux_events[dev][0];
    end = g_aux_events[dev][1];
    ok = true;
  }

  // The second stream's next work waits for everything enqueued on the caller's stream so far.
  bool fork(hipStream_t caller) {
    return hipEventRecord(start, caller) == hipSuccess && hipStreamWaitEvent(stream, start, 0) == hipSuccess;
  }

  // The caller's stream waits for everything enqueued on the second stream so far.
  bool join(hipStream_t caller) {
    return hipEventRecord(end, stream) == hipSuccess && hipStreamWaitEvent(caller, end, 0) == hipSuccess;
  }
};

// How much of each workspace's start is zero for the next call on it, recorded on the host as calls are enqueued
// (calls on one workspace are ordered: they must not overlap). A call needs the zero region of its batch size B
// (topk_zero_bytes(B): the barrier and status words, then B rows' top-k histograms) and leaves exactly that region
// zero, writing anything past it; so a later call whose zero region reaches further first gets the difference
// zero-filled (a fill kernel on its stream). A workspace the record does not hold (its first call, or one dropped
// from the bounded record) gets its whole zero region filled, which is right whatever it holds. A record never
// claims more than is zero: a caller zero-fills a workspace before its first use (so a new workspace at a recorded
// address holds at least the recorded zeros), dsa_workspace_clear records what it clears, and a call that fails
// drops its workspace's record.
struct ZeroRecord {
  int dev;
  const void* ws;
  size_t zero;
};
constexpr int kZeroRecords = 256;
std::mutex g_zero_mu;
ZeroRecord g_zero[kZeroRecords] = {};
int g_zero_next = 0;  // the record replaced next when a new workspace arrives

ZeroRecord* zero_record(int dev, const void* ws) {
  for (ZeroRecord& r : g_zero)
    if (r.ws == ws && r.dev == dev) return &r;
  return nullptr;
}

// A record for a workspace the table does not hold (replacing the oldest one).
ZeroRecord* new_zero_record(int dev, const void* ws) {
  ZeroRecord* r = &g_zero[g_zero_next];
  g_zero_next = (g_zero_next + 1) % kZeroRecords;
  r->dev = dev;
  r->ws = ws;
  return r;
}

// The first `need` bytes of ws zero for the call about to be enqueued on s, and recorded as the call's zero region.
hipError_t ready_zero(void* ws, size_t need, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return hipErrorUnknown;
  std::lock_guard<std::mutex> lock(g_zero_mu);
  ZeroRecord* r = zero_record(dev, ws);
  const size_t have = r ? r->zero : 0;
  if (need > have) {
    const hipError_t e = dsa::launch_fill_zero(static_cast<char*>(ws) + have, need - have, s);
    if (e != hipSuccess) {
      if (r) r->ws = nullptr;
      return e;
    }
  }
  if (!r) r = new_zero_record(dev, ws);
  r->zero = need;
  return hipSuccess;
}

// A call on ws failed: what it left is unknown, so its next call fills its whole zero region.
void drop_zero(const void* ws) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  std::lock_guard<std::mutex> lock(g_zero_mu);
  if (ZeroRecord* r = zero_record(dev, ws)) r->ws = nullptr;
}

// dsa_workspace_clear zeroed the first `bytes` of ws.
void record_cleared(const void* ws, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  std::lock_guard<std::mutex> lock(g_zero_mu);
  ZeroRecord* r = zero_record(dev, ws);
  if (!r) r = new_zero_record(dev, ws);
  r->zero = bytes;
}

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's allocation-free scratch address, looked up on the first call for a device (with that device
// current); its zero region is kept like any workspace's (ready_zero). Null on a HIP error.
void* noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int dsa_abi_version(void) { return DSA_ABI_VERSION; }

int dsa_timing_begin(void* const* events, int pairs) {
  if (pairs < 0 || (pairs > 0 && !events)) return DSA_EINVAL;
  t_timer.events = reinterpret_cast<hipEvent_t*>(const_cast<void**>(events));
  t_timer.pairs = pairs;
  t_timer.launched = 0;
  for (const char*& n : t_timer.names) n = nullptr;
  dsa::g_kernel_timer = &t_timer;
  return DSA_OK;
}

int dsa_timing_end(void) {
  if (!dsa::g_kernel_timer) return 0;
  dsa::g_kernel_timer = nullptr;
  return t_timer.launched;
}

const char* dsa_timing_kernel_name(int k) {
  if (k < 0 || k >= 32 || k >= t_timer.launched || !t_timer.names[k]) return "";
  return t_timer.names[k];
}

const char* dsa_strerror(int s) {
  switch (s) {
    case DSA_OK:
      return "ok";
    case DSA_EINVAL:
      return "invalid argument (null pointer or size out of range)";
    case DSA_EUNSUPPORTED:
      return "unsupported shape";
    case DSA_EWORKSPACE:
      return "workspace too small";
    case DSA_ELAUNCH:
      return "kernel launch failed";
    case DSA_ESCRATCH:
      return "the call needs more scratch than the allocation-free entry point holds (DSA_NOALLOC_SCRATCH_BYTES)";
    default:
      return "unknown status";
  }
}

int dsa_indexer_decode(const void* q_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                       const int32_t* page_table, const int32_t* ctx_len, const float* cand, float* scores, int B,
                       int Hi, int D, int max_pages, int page_size, int num_pages, int score_stride, void* stream) {
  if (!q_bf16 || !w || !k_fp8 || !k_scale || !page_table || !scores) return DSA_EINVAL;
  if (B < 0 || Hi < 1 || max_pages < 1 || page_size < 1 || num_pages < 1 || score_stride < 0) return DSA_EINVAL;
  if (D != 128 || Hi > 64 || page_size % 32) return DSA_EUNSUPPORTED;
  if ((long)score_stride > (long)max_pages * page_size) return DSA_EINVAL;
  if (B == 0 || score_stride == 0) return DSA_OK;
  return status(dsa::launch_indexer_decode(static_cast<const uint16_t*>(q_bf16), w, k_fp8, k_scale, page_table,
                                           ctx_len, cand, scores, nullptr, B, Hi, max_pages, page_size, num_pages,
                                           score_stride, num_cu(), static_cast<hipStream_t>(stream)));
}

int dsa_indexer_decode_bf16(const void* q_bf16, const float* w, const void* k_bf16, const int32_t* page_table,
                            const int32_t* ctx_len, const float* cand, float* scores, int B, int Hi, int D,
                            int max_pages, int page_size, int num_pages, int score_stride, void* stream) {
  if (!q_bf16 || !w || !k_bf16 || !page_table || !scores) return DSA_EINVAL;
  if (B < 0 || Hi < 1 || max_pages < 1 || page_size < 1 || num_pages < 1 || score_stride < 0) return DSA_EINVAL;
  if (D != 128 || Hi > 64) return DSA_EUNSUPPORTED;
  if ((long)score_stride > (long)max_pages * page_size) return DSA_EINVAL;
  if (B == 0 || score_stride == 0) return DSA_OK;
  return status(dsa::launch_indexer_decode_bf16(static_cast<const uint16_t*>(q_bf16), w,
                                                static_cast<const uint16_t*>(k_bf16), page_table, ctx_len, cand,
                                                scores, nullptr, B, Hi, max_pages, page_size, num_pages, score_stride,
                                                static_cast<hipStream_t>(stream)));
}

int dsa_indexer_prefill(const void* q_bf16, const float* w, const void* k, const float* k_scale,
                        const int32_t* npool, float* scores, int N, int Hi, int D, int P, int score_stride,
                        float scale, void* stream) {
  if (!q_bf16 || !w || !k || !npool || !scores) return DSA_EINVAL;
  if (N < 0 || Hi < 1 || P < 1 || score_stride < P || !(scale > 0.0f)) return DSA_EINVAL;
  if (D != 128 || Hi > (k_scale ? 64 : 32)) return DSA_EUNSUPPORTED;
  if (N == 0) return DSA_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (!k_scale)
    return status(dsa::launch_indexer_prefill_bf16k(static_cast<const uint16_t*>(q_bf16), w,
                                                    static_cast<const uint16_t*>(k), npool, scores, N, Hi, P,
                                                    score_stride, scale, nullptr, 0, 0, s));
  return status(dsa::launch_indexer_prefill(static_cast<const uint16_t*>(q_bf16), w, static_cast<const uint8_t*>(k),
                                            k_scale, npool, scores, N, Hi, P, score_stride, scale, nullptr, 0, 0, s));
}

int dsa_indexer_prefill_fp8(const uint8_t* q_fp8, const float* q_scale, const float* w, const uint8_t* k_fp8,
                            const float* k_scale, const int32_t* npool, float* scores, int N, int Hi, int D, int P,
                            int score_stride, float scale, void* stream) {
  if (!q_fp8 || !q_scale || !w || !k_fp8 || !k_scale || !npool || !scores) return DSA_EINVAL;
  if (N < 0 || Hi < 1 || P < 1 || score_stride < P || !(scale > 0.0f)) return DSA_EINVAL;
  if (D != 128 || Hi > 64) return DSA_EUNSUPPORTED;
  if (N == 0) return DSA_OK;
  return status(dsa::launch_indexer_prefill_fp8(q_fp8, q_scale, w, k_fp8, k_scale, npool, scores, N, Hi, P,
                                                score_stride, scale, nullptr, 0, 0, static_cast<hipStream_t>(stream)));
}

size_t dsa_prefill_select_workspace_bytes(int N, int P, int score_stride, int keep, int tile_rows, int own_scores) {
  if (N < 0 || P < 1 || keep < 1 || score_stride < P || tile_rows < 0) return 0;
  return prefill_layout(N, P, score_stride, keep, tile_rows, own_scores != 0).total;
}

int dsa_prefill_select(const void* q, const float* q_scale, const float* w, const void* k, const float* k_scale,
                       const int32_t* npool, float* scores, int64_t* pools, int64_t* cnt, float* vals, void* workspace,
                       size_t workspace_bytes, int N, int Hi, int D, int P, int score_stride, int keep, float scale,
                       int tile_rows, void* stream) {
  if (!q || !w || !k || !npool || !pools || !cnt || !vals || !workspace) return DSA_EINVAL;
  if (N < 0 || Hi < 1 || P < 1 || keep < 1 || score_stride < P || tile_rows < 0 || !(scale > 0.0f))
    return DSA_EINVAL;
  if (q_scale && !k_scale) return DSA_EUNSUPPORTED;  // FP8 queries take FP8 keys
  if (D != 128 || Hi > (k_scale ? 64 : 32)) return DSA_EUNSUPPORTED;
  if (!dsa::topk_supported(P, keep, 1)) return DSA_EUNSUPPORTED;
  const PrefillLayout L = prefill_layout(N, P, score_stride, keep, tile_rows, scores == nullptr);
  if (workspace_bytes < L.total) return DSA_EWORKSPACE;
  if (N == 0) return DSA_OK;
  const hipStream_t a = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const size_t q_row = (size_t)Hi * D * (q_scale ? 1 : 2);  // bytes of one query's heads
  // the generic selection (plan < 0): the indexer writes its sub-block maxima when the sub-blocks are small
  const int gsub = L.plan < 0 ? dsa::topk_two_level_sub(P, keep) : 0;
  const bool gfuse = gsub >= 2 && gsub <= 16;
  int* gidx = reinterpret_cast<int*>(ws + L.gidx_off);
  int* gcnt = reinterpret_cast<int*>(ws + L.gcnt_off);
  // tiles alternate between the caller's stream and the library's second stream, each tile's scores then its
  // selection on one stream: a tile's selection and the boundary of its scores kernel overlap the other stream's
  // tile, and tile t + 2 reuses tile t's buffer set on the same stream (ordered after it without events)
  AuxStream aux(L.plan >= 0 && L.tiles > 1);
  hipError_t e = hipSuccess;
  if (aux.ok && !aux.fork(a)) e = hipErrorUnknown;
  // the generic selection's histograms start at zero: a shorter last tile (here or in an earlier call on this
  // workspace) lays its row meta over the rows a full tile's histograms take
  if (L.plan < 0) e = dsa::launch_fill_zero(workspace, dsa::topk_zero_bytes(L.T), a);
  for (int t = 0; t < L.tiles && e == hipSuccess; ++t) {
    const int r0 = t * L.T, rows = N - r0 < L.T ? N - r0 : L.T, set = t % L.sets;
    const hipStream_t st = aux.ok && set == 1 ? aux.stream : a;
    float* sc = scores ? scores + (size_t)r0 * score_stride
                       : reinterpret_cast<float*>(ws + L.sc_off + (size_t)set * L.sc_bytes);
    float* bm = nullptr;
    int sub_log2 = 0, nb = 0;
    if (L.plan > 0 || gfuse) {
      const int sub = L.plan > 0 ? L.plan : gsub;
      bm = L.plan > 0 ? reinterpret_cast<float*>(ws + L.bm_off + (size_t)set * L.bm_bytes)
                      : dsa::topk_bm_buffer(workspace, rows);
      sub_log2 = __builtin_ctz((unsigned)sub);
      nb = (P + sub - 1) / sub;
    }
    const float* qs = q_scale ? q_scale + (size_t)r0 * Hi : nullptr;
    const char* qt = static_cast<const char*>(q) + (size_t)r0 * q_row;
    const float* wt = w + (size_t)r0 * Hi;
    if (q_scale)
      e = dsa::launch_indexer_prefill_fp8(reinterpret_cast<const uint8_t*>(qt), qs, wt,
                                          static_cast<const uint8_t*>(k), k_scale, npool + r0, sc, rows, Hi, P,
                                          score_stride, scale, bm, sub_log2, nb, st);
    else if (k_scale)
      e = dsa::launch_indexer_prefill(reinterpret_cast<const uint16_t*>(qt), wt, static_cast<const uint8_t*>(k),
                                      k_scale, npool + r0, sc, rows, Hi, P, score_stride, scale, bm, sub_log2, nb,
                                      st);
    else
      e = dsa::launch_indexer_prefill_bf16k(reinterpret_cast<const uint16_t*>(qt), wt,
                                            static_cast<const uint16_t*>(k), npool + r0, sc, rows, Hi, P,
                                            score_stride, scale, bm, sub_log2, nb, st);
    if (e != hipSuccess) break;
    if (L.plan >= 0) {
      int* bidx = reinterpret_cast<int*>(ws + L.bidx_off + (size_t)set * L.bidx_bytes);
      int* bcnt = reinterpret_cast<int*>(ws + L.bcnt_off + (size_t)set * L.bcnt_bytes);
      e = dsa::launch_prefill_tile_topk(sc, score_stride, npool + r0, P, keep, bm, bidx, bcnt,
                                        pools + (size_t)r0 * keep, cnt + r0, vals + (size_t)r0 * keep, rows, st);
    } else {
      e = dsa::launch_prefill_topk(sc, npool + r0, gidx, gcnt, workspace, rows, score_stride, P, keep, gfuse,
                                   pools + (size_t)r0 * keep, cnt + r0, vals + (size_t)r0 * keep, a);
    }
  }
  // the caller's stream waits for everything enqueued on the second stream, whatever failed
  if (aux.ok && !aux.join(a) && e == hipSuccess) e = hipErrorUnknown;
  // a failed generic selection may have left its histograms non-zero: clear them for the next call
  if (e != hipSuccess && L.plan < 0) (void)dsa::launch_fill_zero(workspace, dsa::topk_zero_bytes(L.T), a);
  return status(e);
}

int dsa_cache_write(const void* x, int x_fp32, const int64_t* slots, uint8_t* cache, float* scale, int n_rows, int W,
                    long long num_slots, int per_token_scale, float fp8_max, void* stream) {
  if (!x || !slots || !cache || (per_token_scale && !scale)) return DSA_EINVAL;
  if (n_rows < 0 || num_slots < 1 || !(fp8_max > 0.0f) || !(fp8_max <= 448.0f)) return DSA_EINVAL;
  if (!dsa::cache_write_width_ok(W)) return DSA_EUNSUPPORTED;
  if (n_rows == 0) return DSA_OK;
  return status(dsa::launch_cache_write(x, x_fp32 != 0, slots, cache, scale, n_rows, W, (long)num_slots,
                                        per_token_scale != 0, fp8_max, static_cast<hipStream_t>(stream)));
}

int dsa_pool_keys_write(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                        const int32_t* positions, const int32_t* page_table, int table_shared, int table_pages,
                        const int64_t* slot_mapping, void* pool_key, int n_rows, int kp, int page_size,
                        long long num_slots, void* stream) {
  if (!rows || !ape || !positions || !slot_mapping || !pool_key) return DSA_EINVAL;
  if (n_rows < 0 || table_pages < 1 || page_size < 1 || num_slots < 1 || rows_width < 256) return DSA_EINVAL;
  if (kp < 1 || kp > 8 || (kp & (kp - 1)) || page_size % kp) return DSA_EUNSUPPORTED;
  if (n_rows == 0) return DSA_OK;
  return status(dsa::launch_pool_keys(rows, rows_fp8 != 0, rows_scale, rows_width, ape, positions, page_table,
                                      table_shared != 0, table_pages, slot_mapping, static_cast<uint16_t*>(pool_key),
                                      n_rows, kp, page_size, (long)num_slots, static_cast<hipStream_t>(stream)));
}

int dsa_topk(const float* scores, const int32_t* len, int32_t* idx, int32_t* cnt, void* workspace,
             size_t workspace_bytes, int B, int score_stride, int max_len, int keep, int vis_only, void* stream) {
  if (!scores || !idx || !cnt) return DSA_EINVAL;
  if (B < 0 || score_stride < 1 || keep < 1 || max_len < 0 || max_len > score_stride) return DSA_EINVAL;
  if (!len) max_len = score_stride;
  if (max_len == 0) max_len = 1;
  if (!dsa::topk_supported(max_len, keep, vis_only)) return DSA_EUNSUPPORTED;
  const size_t need = dsa::topk_workspace_bytes(B, max_len, keep);
  if (!workspace || workspace_bytes < need) return DSA_EWORKSPACE;
  if (B == 0) return DSA_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (ready_zero(workspace, dsa::topk_zero_bytes(B), s) != hipSuccess) return DSA_ELAUNCH;
  const int st = status(dsa::launch_topk(scores, len, idx, cnt, workspace, B, score_stride, max_len, keep,
                                         vis_only ? 1 : 0, false, nullptr, 0, 0, 0, nullptr, s));
  if (st != DSA_OK) drop_zero(workspace);
  return st;
}

int dsa_layer_status(void* workspace, int32_t* gave_up, int32_t* two_exchange, int clear, void* stream) {
  if (!gave_up || !two_exchange) return DSA_EINVAL;
  *gave_up = 0;
  *two_exchange = 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = workspace;
  if (!ws) {
    // the current device's allocation-free scratch; none yet: no call has run there
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DSA_ELAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ws = g_scratch_ptr[dev];
    if (!ws) return DSA_OK;
  }
  int32_t words[dsa::WS_SYNC_BYTES / 4];
  if (hipMemcpyAsync(words, ws, sizeof(words), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return DSA_ELAUNCH;
  for (int x = 0; x < 8; ++x) {
    *gave_up += words[x * dsa::WS_SYNC_WORDS + dsa::WS_SYNC_GAVE_UP];
    *two_exchange += words[x * dsa::WS_SYNC_WORDS + dsa::WS_SYNC_TWO_EXCHANGE];
  }
  if (clear) {
    // between calls every other word of the block is zero
    if (dsa::launch_fill_zero(ws, dsa::WS_SYNC_BYTES, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
      return DSA_ELAUNCH;
  }
  return DSA_OK;
}

int dsa_workspace_clear(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15) || (workspace_bytes & 15)) return DSA_EINVAL;
  const int st = status(dsa::launch_fill_zero(workspace, workspace_bytes, static_cast<hipStream_t>(stream)));
  if (st == DSA_OK) record_cleared(workspace, workspace_bytes);
  return st;
}

int dsa_topk_supported(int max_len, int keep, int vis_only) {
  if (max_len < 1 || keep < 1) return 0;
  return dsa::topk_supported(max_len, keep, vis_only) ? 1 : 0;
}

int dsa_topk_mask(const int32_t* idx, const int32_t* cnt, const float* scores, float* mask, int B, int keep, int P,
                  int kp, int tail, void* stream) {
  if (!idx != !cnt || !mask || (tail && !scores)) return DSA_EINVAL;
  if (B < 0 || keep < 1 || P < 1 || kp < 1 || (long)P * kp > 0x7fffffffL) return DSA_EINVAL;
  if (B == 0) return DSA_OK;
  return status(dsa::launch_topk_mask(idx, cnt, scores, mask, B, keep, P, kp, tail != 0,
                                      static_cast<hipStream_t>(stream)));
}

}  // extern "C"

// dsa_sparse_mla_decode with an optional run-time live-row count (n_live: null, or one int on the device; the rows at
// or past it are left unwritten): dsa_sparse_mla_decode and dsa_sparse_mla_slots_n.
static int sparse_mla_decode(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* idx,
                             const int32_t* cnt, const int32_t* page_table, const int32_t* rows, const float* bias,
                             const int32_t* n_live, void* out_bf16, float* out_f32, float* lse, void* workspace,
                             size_t workspace_bytes, int B, int H, int Dqk, int Dv, int keep, int max_pages,
                             int page_size, int num_pages, float scale, int splits, void* stream) {
  if (!q_bf16 || !kv_fp8 || (!out_bf16 && !out_f32)) return DSA_EINVAL;
  const bool token_form = idx != nullptr;
  if (token_form == (rows != nullptr)) return DSA_EINVAL;  // exactly one slot form
  if (token_form && (!cnt || !page_table)) return DSA_EINVAL;
  if (!token_form && !bias) return DSA_EINVAL;
  if (B < 0 || H < 1 || keep < 1 || page_size < 1 || num_pages < 1 || (token_form && max_pages < 1)) return DSA_EINVAL;
  if ((Dqk != 576 && Dqk != 512) || Dv != 512 || H % 16) return DSA_EUNSUPPORTED;
  if ((long)num_pages * page_size > 0x7fffffffL) return DSA_EUNSUPPORTED;
  if (B == 0) return DSA_OK;
  const int sp = effective_splits(resolve_splits(splits, B, H, keep), keep);
  const size_t need = dsa::attention_workspace_bytes(B, H, sp);
  if (need && (!workspace || workspace_bytes < need)) return DSA_EWORKSPACE;
  const bool wide = sp == 1 && dsa::attention_wide_ok(B, H, keep, bias != nullptr, num_cu()) && (token_form || cnt);
  dsa::PoolForm pf{};
  pf.n_live = n_live;
  return status(dsa::launch_sparse_mla(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, idx, cnt, page_table,
                                       rows, bias, static_cast<uint16_t*>(out_bf16), out_f32, lse, workspace, B, H,
                                       Dqk, keep, max_pages, page_size, num_pages, scale, sp,
                                       static_cast<hipStream_t>(stream), pf, wide));
}

extern "C" {

int dsa_sparse_mla_decode(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* idx,
                          const int32_t* cnt, const int32_t* page_table, const int32_t* rows, const float* bias,
                          void* out_bf16, float* out_f32, float* lse, void* workspace, size_t workspace_bytes, int B,
                          int H, int Dqk, int Dv, int keep, int max_pages, int page_size, int num_pages, float scale,
                          int splits, void* stream) {
  return sparse_mla_decode(q_bf16, kv_fp8, kv_scale, idx, cnt, page_table, rows, bias, nullptr, out_bf16, out_f32,
                           lse, workspace, workspace_bytes, B, H, Dqk, Dv, keep, max_pages, page_size, num_pages,
                           scale, splits, stream);
}

int dsa_sparse_mla_slots_n(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* rows,
                           const float* bias, const int32_t* n_live, void* out_bf16, float* out_f32, float* lse,
                           void* workspace, size_t workspace_bytes, int N, int H, int Dqk, int keep,
                           long long num_slots, float scale, int splits, void* stream) {
  if (!rows || !bias || !n_live) return DSA_EINVAL;
  if (num_slots < 1) return DSA_EINVAL;
  if (num_slots > 0x7fffffffLL) return DSA_EUNSUPPORTED;
  return sparse_mla_decode(q_bf16, kv_fp8, kv_scale, nullptr, nullptr, nullptr, rows, bias, n_live, out_bf16, out_f32,
                           lse, workspace, workspace_bytes, N, H, Dqk, 512, keep, 1, 1, (int)num_slots, scale, splits,
                           stream);
}

int dsa_compact_mask(const float* sel, int N, int M, int keep, int64_t* idx, int64_t* cnt, void* stream) {
  if (!sel || !idx || !cnt || N < 0 || M < 1 || keep < 1) return DSA_EINVAL;
  if (N == 0) return DSA_OK;
  return status(dsa::launch_compact_mask(sel, N, M, keep, idx, cnt, static_cast<hipStream_t>(stream)));
}

int dsa_value_order(const int64_t* pools, const int64_t* cnt, const float* vals, int N, int keep,
                    int64_t* out_pools, float* out_vals, void* stream) {
  if (!pools || !cnt || !vals || !out_pools || !out_vals || N < 0 || keep < 1) return DSA_EINVAL;
  if (keep > 8192) return DSA_EUNSUPPORTED;
  if (N == 0) return DSA_OK;
  return status(dsa::launch_value_order(pools, cnt, vals, N, keep, out_pools, out_vals,
                                        static_cast<hipStream_t>(stream)));
}

size_t dsa_slots_compact_workspace_bytes(int B, int H, int NS, int kp, int splits) {
  if (B < 0 || H < 16 || NS < 1 || kp < 1) return 0;
  const int T = NS * kp;
  return align256((size_t)B * T * 4) + align256((size_t)B * 4) +
         align256(dsa::attention_workspace_bytes(B, H, effective_splits(resolve_splits(splits, B, H, T), T)));
}

int dsa_sparse_mla_slots_compact(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                                 const int32_t* rows, const float* bias, void* out_bf16, float* out_f32, float* lse,
                                 void* workspace, size_t workspace_bytes, int B, int H, int Dqk, int NS, int kp,
                                 long long num_slots, float scale, int splits, void* stream) {
  if (!q_bf16 || !kv_fp8 || !rows || !bias || (!out_bf16 && !out_f32)) return DSA_EINVAL;
  if (B < 0 || H < 1 || NS < 1 || kp < 1 || num_slots < kp || num_slots % kp) return DSA_EINVAL;
  if ((Dqk != 576 && Dqk != 512) || H % 16) return DSA_EUNSUPPORTED;
  if (num_slots > 0x7fffffffL || (long long)NS * kp > 0x7fffffffL) return DSA_EUNSUPPORTED;
  if (B == 0) return DSA_OK;
  const int T = NS * kp;
  const size_t need = dsa_slots_compact_workspace_bytes(B, H, NS, kp, splits);
  if (!workspace || workspace_bytes < need) return DSA_EWORKSPACE;
  auto* s = static_cast<hipStream_t>(stream);
  char* p = static_cast<char*>(workspace);
  int* tok = reinterpret_cast<int*>(p);
  int* tcnt = reinterpret_cast<int*>(p + align256((size_t)B * T * 4));
  void* aws = p + align256((size_t)B * T * 4) + align256((size_t)B * 4);
  if (dsa::launch_compact_slots(rows, bias, B, NS, kp, (int)(num_slots / kp), tok, tcnt, s) != hipSuccess)
    return DSA_ELAUNCH;
  // the compacted rows + count form; a row with no visible token attends its list's kp entries, all masked
  const int sp = effective_splits(resolve_splits(splits, B, H, T), T);
  dsa::PoolForm pf{};
  pf.empty_n = kp;
  const bool wide = sp == 1 && dsa::attention_wide_ok(B, H, T, false, num_cu());
  return status(dsa::launch_sparse_mla(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, nullptr, tcnt,
                                       nullptr, tok, nullptr, static_cast<uint16_t*>(out_bf16), out_f32, lse, aws, B,
                                       H, Dqk, T, 1, 1, (int)num_slots, scale, sp, s, pf, wide));
}

int dsa_token_rows(const int32_t* idx, const int32_t* cnt, const int32_t* page_table, int32_t* rows, float* bias,
                   int B, int keep, int max_pages, int page_size, int num_pages, void* stream) {
  if (!idx || !cnt || !page_table || !rows) return DSA_EINVAL;
  if (B < 0 || keep < 1 || max_pages < 1 || page_size < 1 || num_pages < 1) return DSA_EINVAL;
  if (B == 0) return DSA_OK;
  return status(dsa::launch_token_rows(idx, cnt, page_table, rows, bias, B, keep, max_pages, page_size, num_pages,
                                       static_cast<hipStream_t>(stream)));
}

int dsa_pool_slots(const int32_t* pools, const int32_t* cnt, const int32_t* npool, const int32_t* positions,
                   const int32_t* table, int table_shared, int32_t* rows, float* bias, int N, int keep, int n_slots,
                   int table_pages, int page_size, int kp, void* stream) {
  if (!pools || !cnt || !npool || !positions || !table || !rows || !bias) return DSA_EINVAL;
  if (N < 0 || keep < 1 || n_slots < keep + 1 || table_pages < 1 || kp < 1) return DSA_EINVAL;
  const int ppp = page_size / kp;
  if (page_size % kp || ppp < 1 || (ppp & (ppp - 1))) return DSA_EINVAL;
  if (N == 0) return DSA_OK;
  return status(dsa::launch_pool_slots(pools, cnt, npool, positions, table, table_shared != 0, rows, bias, N, keep,
                                       n_slots, table_pages, page_size, kp, static_cast<hipStream_t>(stream)));
}

size_t dsa_workspace_bytes(int kind, int B, int H, int keep, int max_len, int splits) {
  if (B < 0 || keep < 1) return 0;
  size_t t = 0, a = 0;
  if (kind == DSA_WS_TOPK || kind == DSA_WS_LAYER) t = dsa::topk_workspace_bytes(B, max_len, keep);
  if (kind == DSA_WS_LAYER) t = align256(t) + layer_rows_bytes(B, keep);
  if (kind == DSA_WS_ATTENTION || kind == DSA_WS_LAYER) {
    if (H < 16) return align256(t);
    const int sp = effective_splits(resolve_splits(splits, B, H, keep), keep);
    a = dsa::attention_workspace_bytes(B, H, sp);
  }
  size_t total = align256(t) + align256(a);
  if (kind == DSA_WS_LAYER) {
    // the one-launch layer's layout shares the zero region and needs its own rest; the separate kernels' XCD-local
    // attention takes the attention's place
    const size_t f = dsa::fused_layer_bytes(dsa::topk_zero_bytes(B), B, H, keep);
    const size_t x = align256(t) + align256(dsa::attend_xcd_bytes(B, H, keep));
    // rows past 32,768 tokens: the selection, attention and combine in one launch, its lists past the attention's
    const size_t lg = align256(t) + align256(dsa::long_attend_bytes(B, H, keep, max_len));
    total = f > total ? f : total;
    total = x > total ? x : total;
    total = lg > total ? lg : total;
  }
  return total;
}

int dsa_default_splits(int B, int H, int keep) {
  if (B < 1 || H < 16 || keep < 1) return 1;
  return effective_splits(resolve_splits(0, B, H, keep), keep);
}

static int layer_chain(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                       const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                       const int32_t* ctx_len, float* scores, int32_t* idx, int32_t* cnt, void* out_bf16, float* lse,
                       void* workspace, size_t workspace_bytes, int B, int Hi, int H, int max_pages, int page_size,
                       int num_pages, int score_stride, int max_len, int keep, float scale, int splits,
                       void* stream);

static int pooled_layer(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                        const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table, const int32_t* npool,
                        const int32_t* positions, float* scores, int32_t* pools, int32_t* cnt, void* out_bf16,
                        float* lse, void* workspace, int B, int Hi, int H, int Dqk, int max_pages, int page_size,
                        int num_pages, int kp, int keep, float scale, int splits, int stride, hipStream_t s);
// The decode layer's checks, shared by its forms (every check before the first launch: a rejected call writes
// nothing); need_ws: the caller passes a workspace (the allocation-free form checks its scratch's size itself).
static int layer_checks(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                        const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                        const int32_t* ctx_len, float* scores, int32_t* idx, int32_t* cnt, void* out_bf16,
                        void* workspace, size_t workspace_bytes, int B, int Hi, int H, int max_pages, int page_size,
                        int num_pages, int score_stride, int max_len, int keep, int splits, bool need_ws = true) {
  if (!q_idx_bf16 || !w || !k_fp8 || !k_scale || !page_table || !ctx_len || !scores || !idx || !cnt)
    return DSA_EINVAL;
  if (need_ws && !workspace) return DSA_EINVAL;
  if (!q_bf16 || !kv_fp8 || !out_bf16) return DSA_EINVAL;
  if (B < 0 || Hi < 1 || H < 1 || max_pages < 1 || page_size < 1 || num_pages < 1 || keep < 1) return DSA_EINVAL;
  if (max_len < 1 || max_len > score_stride || (long)score_stride > (long)max_pages * page_size) return DSA_EINVAL;
  if (Hi > 64 || page_size % 32 || H % 16) return DSA_EUNSUPPORTED;
  if ((long)num_pages * page_size > 0x7fffffffL) return DSA_EUNSUPPORTED;
  if (!dsa::topk_supported(max_len, keep, 1)) return DSA_EUNSUPPORTED;
  if (need_ws && workspace_bytes < dsa_workspace_bytes(DSA_WS_LAYER, B, H, keep, max_len, splits))
    return DSA_EWORKSPACE;
  return DSA_OK;
}

int dsa_decode_layer(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                     const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                     const int32_t* ctx_len, float* scores, int32_t* idx, int32_t* cnt, void* out_bf16, float* lse,
                     void* workspace, size_t workspace_bytes, int B, int Hi, int H, int max_pages, int page_size,
                     int num_pages, int score_stride, int max_len, int keep, float scale, int splits, void* stream) {
  const int st = layer_checks(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len, scores,
                              idx, cnt, out_bf16, workspace, workspace_bytes, B, Hi, H, max_pages, page_size,
                              num_pages, score_stride, max_len, keep, splits);
  if (st != DSA_OK || B == 0) return st;
  if (!dsa::fused_layer_ok(num_cu(), Hi, H, max_len, keep, page_size, score_stride))
    return dsa_decode_layer_chain(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len,
                                  scores, idx, cnt, out_bf16, lse, workspace, workspace_bytes, B, Hi, H, max_pages,
                                  page_size, num_pages, score_stride, max_len, keep, scale, splits, stream);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (ready_zero(workspace, dsa::topk_zero_bytes(B), s) != hipSuccess) return DSA_ELAUNCH;
  const int r = status(dsa::launch_decode_fused(
      static_cast<const uint16_t*>(q_idx_bf16), w, k_fp8, k_scale, static_cast<const uint16_t*>(q_bf16), kv_fp8,
      kv_scale, page_table, ctx_len, scores, idx, cnt, static_cast<uint16_t*>(out_bf16), lse, workspace,
      dsa::topk_zero_bytes(B), B, Hi, H, max_pages, page_size, num_pages, score_stride, keep, scale, s));
  if (r != DSA_OK) drop_zero(workspace);
  return r;
}

int dsa_decode_layer_chain(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                           const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                           const int32_t* page_table, const int32_t* ctx_len, float* scores, int32_t* idx,
                           int32_t* cnt, void* out_bf16, float* lse, void* workspace, size_t workspace_bytes, int B,
                           int Hi, int H, int max_pages, int page_size, int num_pages, int score_stride, int max_len,
                           int keep, float scale, int splits, void* stream) {
  const int st = layer_checks(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len, scores,
                              idx, cnt, out_bf16, workspace, workspace_bytes, B, Hi, H, max_pages, page_size,
                              num_pages, score_stride, max_len, keep, splits);
  if (st != DSA_OK || B == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ready_zero(workspace, dsa::topk_zero_bytes(B), s) != hipSuccess) return DSA_ELAUNCH;
  const int r = layer_chain(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len, scores, idx,
                            cnt, out_bf16, lse, workspace, workspace_bytes, B, Hi, H, max_pages, page_size, num_pages,
                            score_stride, max_len, keep, scale, splits, stream);
  if (r != DSA_OK) drop_zero(workspace);
  return r;
}

}  // extern "C"

// The separate kernels of dsa_decode_layer_chain, after its checks and with the workspace's zero region ready.
static int layer_chain(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                       const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                       const int32_t* ctx_len, float* scores, int32_t* idx, int32_t* cnt, void* out_bf16, float* lse,
                       void* workspace, size_t workspace_bytes, int B, int Hi, int H, int max_pages, int page_size,
                       int num_pages, int score_stride, int max_len, int keep, float scale, int splits,
                       void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t t_need = align256(dsa::topk_workspace_bytes(B, max_len, keep));
  // the indexer accumulates the top-k's first-level histogram (the workspace's first region): flat rows, and a few
  // long rows (the long selection; the long-row indexer); otherwise long rows take the two-level selection, the
  // long-row indexer writing its first-level sub-block maxima (sub-blocks of up to 32)
  const bool flat = max_len <= 32 * 1024;
  const bool long_sel = !flat && dsa::topk_long_rows(B, max_len);
  const bool fused_hist = flat || long_sel;
  const int sub = fused_hist ? 0 : dsa::topk_two_level_sub(max_len, keep);
  const bool fused_bm = sub >= 2 && sub <= 32;
  int* hist = fused_hist ? dsa::ws_hist(workspace) : nullptr;
  // long rows through the one-launch selection and attention: for rows past 524,288 tokens the indexer also writes
  // the maxima of the rows' 32-key tiles into that launch's workspace
  const bool la = long_sel && splits == 0 && dsa::long_attend_ok(num_cu(), H, keep, max_len, score_stride);
  char* lws = static_cast<char*>(workspace) + t_need + layer_rows_bytes(B, keep);
  float* tmax = la && dsa::long_attend_tiles(max_len) ? dsa::long_attend_tmax(lws, B, H, keep, max_len) : nullptr;
  hipError_t e;
  if (flat)
    e = dsa::launch_indexer_decode(static_cast<const uint16_t*>(q_idx_bf16), w, k_fp8, k_scale, page_table, ctx_len,
                                   nullptr, scores, hist, B, Hi, max_pages, page_size, num_pages, score_stride,
                                   num_cu(), s);
  else
    e = dsa::launch_indexer_decode_long(static_cast<const uint16_t*>(q_idx_bf16), w, k_fp8, k_scale, page_table,
                                        ctx_len, scores,
                                        tmax ? tmax : fused_bm ? dsa::topk_bm_buffer(workspace, B) : nullptr,
                                        tmax ? 5 : fused_bm ? __builtin_ctz((unsigned)sub) : 0,
                                        tmax ? dsa::long_attend_ntile(max_len) : fused_bm ? (max_len + sub - 1) / sub : 0,
                                        hist, B, Hi, max_pages, page_size, num_pages, score_stride, num_cu(), s);
  if (e != hipSuccess) {
    if (hist) dsa::launch_fill_zero(hist, dsa::topk_hist_bytes(B), s);  // a partial histogram may be in
    return DSA_ELAUNCH;
  }
  if (la) {
    // the long rows' selection, attention and combine in one launch over the indexer's scores, histograms and tile
    // maxima
    e = dsa::launch_decode_long_attend(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, page_table, ctx_len,
                                       scores, score_stride, hist, idx, cnt, static_cast<uint16_t*>(out_bf16), lse,
                                       lws, static_cast<int*>(workspace), B, H, max_pages, page_size, num_pages, keep,
                                       scale, max_len, s);
    if (e != hipSuccess) {
      dsa::launch_fill_zero(dsa::ws_hist(workspace), dsa::topk_hist_bytes(B), s);  // (as below)
      return DSA_ELAUNCH;
    }
    return DSA_OK;
  }
  // with the histogram from the indexer the top-k also resolves the selected positions to cache slots, so the
  // attention reads slot ids directly (one dependent load round fewer)
  int* rows = fused_hist ? reinterpret_cast<int*>(static_cast<char*>(workspace) + t_need) : nullptr;
  e = dsa::launch_topk(scores, ctx_len, idx, cnt, workspace, B, score_stride, max_len, keep, 1, fused_hist,
                       page_table, max_pages, page_size, num_pages, rows, s, fused_bm);
  if (e != hipSuccess) {
    // the indexer has added into the histograms, which the top-k would have cleared: clear them here, so that the
    // workspace stays usable (if this launch fails too, dsa_workspace_clear must run before the next call)
    dsa::launch_fill_zero(dsa::ws_hist(workspace), dsa::topk_hist_bytes(B), s);
    return DSA_ELAUNCH;
  }
  char* aws = static_cast<char*>(workspace) + t_need + layer_rows_bytes(B, keep);
  const size_t aws_bytes = workspace_bytes - t_need - layer_rows_bytes(B, keep);
  // the default split count on a GPU of 8 XCDs x 32 CUs: the one-launch layer's attention and combine as a launch of
  // their own (XCD-local, bf16 split outputs), over the slot rows (flat rows) or the positions through the page table
  if (splits == 0 && dsa::attend_xcd_ok(num_cu(), H, keep))
    return status(dsa::launch_decode_attend(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, rows,
                                            rows ? nullptr : idx, page_table, cnt, static_cast<uint16_t*>(out_bf16),
                                            lse, aws, static_cast<int*>(workspace), B, H, max_pages, page_size,
                                            num_pages, keep, scale, s));
  if (!rows)
    return dsa_sparse_mla_decode(q_bf16, kv_fp8, kv_scale, idx, cnt, page_table, nullptr, nullptr, out_bf16, nullptr,
                                 lse, aws, aws_bytes, B, H, 576, 512, keep, max_pages, page_size, num_pages, scale,
                                 splits, stream);
  const int sp = effective_splits(resolve_splits(splits, B, H, keep), keep);
  return status(dsa::launch_sparse_mla(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, nullptr, cnt, nullptr,
                                       rows, nullptr, static_cast<uint16_t*>(out_bf16), nullptr, lse, aws, B, H, 576,
                                       keep, max_pages, page_size, num_pages, scale, sp, s));
}

extern "C" {

int dsa_decode_layer_noalloc(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                             const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                             const int32_t* page_table, const int32_t* ctx_len, float* scores, int32_t* idx,
                             int32_t* cnt, void* out_bf16, float* lse, int B, int Hi, int H, int max_pages,
                             int page_size, int num_pages, int score_stride, int max_len, int keep, float scale,
                             int splits, void* stream) {
  // every check first (no HIP call, no fill enqueued, for a refused call): the layer's own, then its workspace
  // against the scratch
  const int st = layer_checks(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len, scores,
                              idx, cnt, out_bf16, nullptr, 0, B, Hi, H, max_pages, page_size, num_pages, score_stride,
                              max_len, keep, splits, false);
  if (st != DSA_OK) return st;
  const size_t need = dsa_workspace_bytes(DSA_WS_LAYER, B, H, keep, max_len, splits);
  if (need == 0 || need > DSA_NOALLOC_SCRATCH_BYTES) return DSA_ESCRATCH;
  if (B == 0) return DSA_OK;
  void* ws = noalloc_scratch();
  if (!ws) return DSA_ELAUNCH;
  return dsa_decode_layer(q_idx_bf16, w, k_fp8, k_scale, q_bf16, kv_fp8, kv_scale, page_table, ctx_len, scores, idx,
                          cnt, out_bf16, lse, ws, DSA_NOALLOC_SCRATCH_BYTES, B, Hi, H, max_pages, page_size,
                          num_pages, score_stride, max_len, keep, scale, splits, stream);
}

size_t dsa_sparse_mla_pooled_workspace_bytes(int B, int H, int keep, int kp, int splits) {
  if (B < 0 || H < 16 || keep < 1 || kp < 2) return 0;
  const int keep_sel = kp * keep;  // the selected pools' token slots; the tail comes on top
  return align256(dsa::attention_workspace_bytes(B, H, effective_splits(resolve_splits(splits, B, H, keep_sel),
                                                                          keep_sel)));
}

int dsa_sparse_mla_pooled(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* pools,
                          const int32_t* cnt, const int32_t* npool, const int32_t* positions, const int32_t* page_table,
                          void* out_bf16, float* out_f32, float* lse, void* workspace, size_t workspace_bytes, int B,
                          int H, int Dqk, int keep, int kp, int max_pages, int page_size, int num_pages, float scale,
                          int splits, void* stream) {
  if (!q_bf16 || !kv_fp8 || !pools || !cnt || !npool || !positions || !page_table) return DSA_EINVAL;
  if (!out_bf16 && !out_f32) return DSA_EINVAL;
  if (B < 0 || H < 1 || keep < 1 || max_pages < 1 || page_size < 1 || num_pages < 1) return DSA_EINVAL;
  if (kp < 2 || kp > 8 || (kp & (kp - 1)) || page_size % kp) return DSA_EUNSUPPORTED;
  if ((Dqk != 576 && Dqk != 512) || H % 16) return DSA_EUNSUPPORTED;
  if ((long)num_pages * page_size > 0x7fffffffL) return DSA_EUNSUPPORTED;
  if (B == 0) return DSA_OK;
  const int keep_sel = kp * keep;  // the selected pools' token slots; the tail comes on top
  const int sp = effective_splits(resolve_splits(splits, B, H, keep_sel), keep_sel);
  const size_t need = dsa::attention_workspace_bytes(B, H, sp);
  if (need && (!workspace || workspace_bytes < need)) return DSA_EWORKSPACE;
  const dsa::PoolForm pf = {__builtin_ctz((unsigned)kp), keep, npool, positions, 0, 0, nullptr};
  const bool wide = sp == 1 && dsa::attention_wide_ok(B, H, keep_sel + kp, false, num_cu());
  return status(dsa::launch_sparse_mla(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, pools, cnt, page_table,
                                       nullptr, nullptr, static_cast<uint16_t*>(out_bf16), out_f32, lse, workspace, B,
                                       H, Dqk, keep_sel, max_pages, page_size, num_pages, scale, sp,
                                       static_cast<hipStream_t>(stream), pf, wide));
}

size_t dsa_pooled_workspace_bytes(int B, int H, int keep, int max_len, int kp, int splits) {
  if (B < 0 || H < 16 || keep < 1 || max_len < 1 || kp < 2) return 0;
  const int keep_sel = kp * keep;
  const int sp = effective_splits(resolve_splits(splits, B, H, keep_sel), keep_sel);
  // the split attention's workspace, or the XCD-local attention launch's (split outputs and their (max, sum))
  const size_t t = align256(dsa::topk_workspace_bytes(B, max_len, keep));
  const size_t a = align256(dsa::attention_workspace_bytes(B, H, sp));
  const size_t x = align256(dsa::attend_xcd_bytes(B, H, keep_sel));
  // the one-launch form's layout shares the zero region and needs its own rest (key lists, split outputs)
  const size_t f = align256(dsa::fused_pooled_bytes(dsa::topk_zero_bytes(B), B, H));
  const size_t chain = t + (a > x ? a : x);
  return f > chain ? f : chain;
}

// The pooled layer's checks (every check before the first launch) and its pool stride; DSA_OK or a status.
static int pooled_checks(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                         const uint8_t* kv_fp8, const int32_t* page_table, const int32_t* npool,
                         const int32_t* positions, float* scores, int32_t* pools, int32_t* cnt, void* out_bf16,
                         void* workspace, size_t workspace_bytes, int B, int Hi, int H, int Dqk, int max_pages,
                         int page_size, int num_pages, int kp, int keep, int splits, int* stride_out) {
  if (!q_idx_bf16 || !w || !pool_key_bf16 || !q_bf16 || !kv_fp8 || !page_table || !npool || !positions || !scores ||
      !pools || !cnt || !out_bf16 || !workspace)
    return DSA_EINVAL;
  if (B < 0 || Hi < 1 || H < 1 || max_pages < 1 || page_size < 1 || num_pages < 1 || keep < 1) return DSA_EINVAL;
  if (kp < 2 || kp > 8 || (kp & (kp - 1)) || page_size % kp) return DSA_EUNSUPPORTED;
  const int ppp = page_size / kp;  // pools per page
  const long stride_l = (long)max_pages * ppp;
  if (stride_l > 0x7fffffffL || (long)num_pages * page_size > 0x7fffffffL) return DSA_EUNSUPPORTED;
  const int stride = (int)stride_l;
  if (Hi > 64 || H % 16 || (Dqk != 512 && Dqk != 576)) return DSA_EUNSUPPORTED;
  if (!dsa::topk_supported(stride, keep, 1)) return DSA_EUNSUPPORTED;
  if (workspace_bytes < dsa_pooled_workspace_bytes(B, H, keep, stride, kp, splits)) return DSA_EWORKSPACE;
  *stride_out = stride;
  return DSA_OK;
}

// The pooled layer in one launch when fused_pooled_ok holds (pkw: the step's pool-key write in the same launch),
// otherwise the write's own kernel (pkw) and the separate kernels.
static int pooled_layer_or_step(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                                const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                                const int32_t* npool, const int32_t* positions, float* scores, int32_t* pools,
                                int32_t* cnt, void* out_bf16, float* lse, void* workspace, size_t workspace_bytes,
                                int B, int Hi, int H, int Dqk, int max_pages, int page_size, int num_pages, int kp,
                                int keep, float scale, int splits, const dsa::PoolKeyWrite* pkw, void* stream) {
  int stride = 0;
  const int st = pooled_checks(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, page_table, npool, positions, scores,
                               pools, cnt, out_bf16, workspace, workspace_bytes, B, Hi, H, Dqk, max_pages, page_size,
                               num_pages, kp, keep, splits, &stride);
  if (st != DSA_OK || B == 0) return st;
  if (splits != 0 || !dsa::fused_pooled_ok(num_cu(), Hi, H, Dqk, stride, kp, page_size, keep)) {
    if (pkw) {
      const int r = dsa_pool_keys_write(pkw->rows, pkw->rows_fp8, pkw->rows_scale, pkw->rows_width, pkw->ape,
                                        positions, page_table, 0, max_pages, pkw->slot_mapping,
                                        const_cast<void*>(pool_key_bf16), B, kp, page_size,
                                        (long long)num_pages * page_size, stream);
      if (r != DSA_OK) return r;
    }
    return dsa_pooled_decode_layer_chain(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, kv_scale, page_table, npool,
                                         positions, scores, pools, cnt, out_bf16, lse, workspace, workspace_bytes, B,
                                         Hi, H, Dqk, max_pages, page_size, num_pages, kp, keep, scale, splits, stream);
  }
  if (pkw && !dsa::fused_step_ok(kp)) {
    // the write's own kernel, then the layer's one launch
    const int r = dsa_pool_keys_write(pkw->rows, pkw->rows_fp8, pkw->rows_scale, pkw->rows_width, pkw->ape, positions,
                                      page_table, 0, max_pages, pkw->slot_mapping, const_cast<void*>(pool_key_bf16),
                                      B, kp, page_size, (long long)num_pages * page_size, stream);
    if (r != DSA_OK) return r;
    pkw = nullptr;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ready_zero(workspace, dsa::topk_zero_bytes(B), s) != hipSuccess) return DSA_ELAUNCH;
  const int r = status(dsa::launch_decode_fused_pooled(
      static_cast<const uint16_t*>(q_idx_bf16), w, static_cast<const uint16_t*>(pool_key_bf16),
      static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, page_table, npool, positions, scores, pools, cnt,
      static_cast<uint16_t*>(out_bf16), lse, workspace, dsa::topk_zero_bytes(B), B, Hi, H, max_pages, page_size,
      num_pages, kp, keep, scale, pkw, s));
  if (r != DSA_OK) drop_zero(workspace);
  return r;
}

int dsa_pooled_decode_layer(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                            const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                            const int32_t* npool, const int32_t* positions, float* scores, int32_t* pools,
                            int32_t* cnt, void* out_bf16, float* lse, void* workspace, size_t workspace_bytes, int B,
                            int Hi, int H, int Dqk, int max_pages, int page_size, int num_pages, int kp, int keep,
                            float scale, int splits, void* stream) {
  return pooled_layer_or_step(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, kv_scale, page_table, npool, positions,
                              scores, pools, cnt, out_bf16, lse, workspace, workspace_bytes, B, Hi, H, Dqk, max_pages,
                              page_size, num_pages, kp, keep, scale, splits, nullptr, stream);
}

int dsa_pooled_decode_step(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                           const int64_t* slot_mapping, const void* q_idx_bf16, const float* w, void* pool_key_bf16,
                           const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                           const int32_t* page_table, const int32_t* npool, const int32_t* positions, float* scores,
                           int32_t* pools, int32_t* cnt, void* out_bf16, float* lse, void* workspace,
                           size_t workspace_bytes, int B, int Hi, int H, int Dqk, int max_pages, int page_size,
                           int num_pages, int kp, int keep, float scale, int splits, void* stream) {
  if (!rows || !ape || !slot_mapping) return DSA_EINVAL;
  if (rows_width < 256) return DSA_EINVAL;
  const dsa::PoolKeyWrite pkw{rows, rows_scale, ape, slot_mapping, rows_width, rows_fp8 != 0};
  return pooled_layer_or_step(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, kv_scale, page_table, npool, positions,
                              scores, pools, cnt, out_bf16, lse, workspace, workspace_bytes, B, Hi, H, Dqk, max_pages,
                              page_size, num_pages, kp, keep, scale, splits, &pkw, stream);
}

int dsa_pooled_decode_layer_chain(const void* q_idx_bf16, const float* w, const void* pool_key_bf16,
                                  const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                                  const int32_t* page_table, const int32_t* npool, const int32_t* positions,
                                  float* scores, int32_t* pools, int32_t* cnt, void* out_bf16, float* lse,
                                  void* workspace, size_t workspace_bytes, int B, int Hi, int H, int Dqk,
                                  int max_pages, int page_size, int num_pages, int kp, int keep, float scale,
                                  int splits, void* stream) {
  int stride = 0;
  const int st = pooled_checks(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, page_table, npool, positions, scores,
                               pools, cnt, out_bf16, workspace, workspace_bytes, B, Hi, H, Dqk, max_pages, page_size,
                               num_pages, kp, keep, splits, &stride);
  if (st != DSA_OK || B == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ready_zero(workspace, dsa::topk_zero_bytes(B), s) != hipSuccess) return DSA_ELAUNCH;
  const int r = pooled_layer(q_idx_bf16, w, pool_key_bf16, q_bf16, kv_fp8, kv_scale, page_table, npool, positions,
                             scores, pools, cnt, out_bf16, lse, workspace, B, Hi, H, Dqk, max_pages, page_size,
                             num_pages, kp, keep, scale, splits, stride, s);
  if (r != DSA_OK) drop_zero(workspace);
  return r;
}

}  // extern "C"

// The kernels of dsa_pooled_decode_layer, after its checks and with the workspace's zero region ready.
static int pooled_layer(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                        const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table, const int32_t* npool,
                        const int32_t* positions, float* scores, int32_t* pools, int32_t* cnt, void* out_bf16,
                        float* lse, void* workspace, int B, int Hi, int H, int Dqk, int max_pages, int page_size,
                        int num_pages, int kp, int keep, float scale, int splits, int stride, hipStream_t s) {
  const int ppp = page_size / kp;  // pools per page
  const size_t t_need = align256(dsa::topk_workspace_bytes(B, stride, keep));
  // flat rows: the indexer accumulates the top-k's first-level histogram (the workspace's first region)
  const bool fused_hist = stride <= 32 * 1024;
  hipError_t e = dsa::launch_indexer_decode_bf16(static_cast<const uint16_t*>(q_idx_bf16), w,
                                                 static_cast<const uint16_t*>(pool_key_bf16), page_table, npool,
                                                 nullptr, scores, fused_hist ? dsa::ws_hist(workspace) : nullptr,
                                                 B, Hi, max_pages, ppp, num_pages, stride, s);
  if (e != hipSuccess) return DSA_ELAUNCH;
  e = dsa::launch_topk(scores, npool, pools, cnt, workspace, B, stride, stride, keep, 1, fused_hist, nullptr, 0, 0, 0,
                       nullptr, s);
  if (e != hipSuccess) {
    // the histograms the indexer added into stay zero for the next call (as in dsa_decode_layer)
    dsa::launch_fill_zero(dsa::ws_hist(workspace), dsa::topk_hist_bytes(B), s);
    return DSA_ELAUNCH;
  }
  const int keep_sel = kp * keep;  // the selected pools' token slots; the tail comes on top
  // the default split count on a GPU of 8 XCDs x 32 CUs, 512-wide rows: the attention and combine in one XCD-local
  // launch (the separate kernels' form of the one-launch layer's last stages), the tail in the split of the last
  // selected token; the barrier words are the workspace's first bytes
  if (splits == 0 && dsa::attend_xcd_pooled_ok(num_cu(), H, Dqk, keep_sel))
    return status(dsa::launch_decode_attend_pooled(
        static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, pools, cnt, npool, positions, page_table,
        static_cast<uint16_t*>(out_bf16), lse, static_cast<char*>(workspace) + t_need, static_cast<int*>(workspace), B,
        H, max_pages, page_size, num_pages, keep, __builtin_ctz((unsigned)kp), scale, s));
  const int sp = effective_splits(resolve_splits(splits, B, H, keep_sel), keep_sel);
  const dsa::PoolForm pf = {__builtin_ctz((unsigned)kp), keep, npool, positions, 0, 0, nullptr};
  return status(dsa::launch_sparse_mla(static_cast<const uint16_t*>(q_bf16), kv_fp8, kv_scale, pools, cnt, page_table,
                                       nullptr, nullptr, static_cast<uint16_t*>(out_bf16), nullptr, lse,
                                       static_cast<char*>(workspace) + t_need, B, H, Dqk, keep_sel, max_pages,
                                       page_size, num_pages, scale, sp, s, pf));
}
