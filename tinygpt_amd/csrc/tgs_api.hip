// tgs_api.hip -- host side of the C ABI declared in include/tgs_sampler.h.
//
// The handle owns the split-row workspace (chunk candidate lists), the
// speculative workspace and the mask table.  Calls validate host-visible
// arguments, pick the kernel variant from the batch hint and the split
// (chunks per row) from the batch size, size the dynamic LDS and launch on
// the caller's stream (chunk kernel, then the merge kernel when rows are
// split).  Nothing here allocates during tgs_sample.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "tgs_device.h"
#include "tgs_kernels.h"

struct tgs_ctx {
  int device = 0;
  int max_batch = 0, max_vocab = 0, max_hist = 0;
  int num_cu = 256;
  size_t lds_limit = 65536;
  unsigned long long* ws = nullptr;
  int* ws_cnt = nullptr;
  int ws_rows = 0;  // chunk lists of KMAX entries the workspace holds
  unsigned* k64_cnt = nullptr;  // fused kernel exchange lines (arrival counter, epoch, count words), one per row
  unsigned long long* k64_lists = nullptr;  // fused kernel chunk lists, [max_batch * kMaxSplit][64]
  unsigned long long* k64_keys = nullptr;   // fused kernel bound-exchange keys, [max_batch][K64_KEYS]
  uint32_t* mask_table = nullptr;
  int n_states = 0, mask_vocab = 0, mask_words = 0;
  void* mask_stage = nullptr;  // tgs_mask_table_update staging (grown on demand)
  size_t mask_stage_bytes = 0;
  float* spec_blk_m = nullptr;             // speculative workspace (tgs_reserve_spec)
  unsigned long long* spec_blk_q = nullptr;
  unsigned long long* spec_blk_w = nullptr;
  void* spec_state = nullptr;
  int spec_b = 0, spec_k = -1, spec_nbs = 0;
  std::string err;
};

namespace {

constexpr int kMaxVocab = 262144;  // 256 speculative blocks of 1024 ids
constexpr int kMaxHist = 4096;
constexpr int kMaxSplit = 16;

struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int fail(tgs_ctx* h, int code, const std::string& msg) {
  if (h) h->err = msg;
  return code;
}

int hip_fail(tgs_ctx* h, hipError_t e, const char* what) {
  return fail(h, TGS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}
int log2i(int x) {
  int l = 0;
  while ((1 << l) < x) l++;
  return l;
}

void free_spec(tgs_ctx* h) {
  if (h->spec_blk_m) (void)hipFree(h->spec_blk_m);
  if (h->spec_blk_q) (void)hipFree(h->spec_blk_q);
  if (h->spec_blk_w) (void)hipFree(h->spec_blk_w);
  if (h->spec_state) (void)hipFree(h->spec_state);
  h->spec_blk_m = nullptr;
  h->spec_blk_q = nullptr;
  h->spec_blk_w = nullptr;
  h->spec_state = nullptr;
  h->spec_b = 0;
  h->spec_k = -1;
  h->spec_nbs = 0;
}

// Chunks per row of the fused top_k <= 64 kernel: about one workgroup per CU
// (chunks of at least 2048 ids), never fewer chunks than a workgroup's
// capacity requires, at most K64_MAX_SPLIT.  TGS_SPLIT sets the split
// (tuning, tests).
constexpr int kMaxSplitK64 = tgs::K64_MAX_SPLIT;
int choose_split_k64(int num_cu, int B, int V, int dt) {
  const int ch = tgs::k64_chunk_ids(dt);
  const int smin = (V + ch - 1) / ch;
  int S;
  const char* env = std::getenv("TGS_SPLIT");
  if (env && std::atoi(env) > 0) {
    S = std::min(std::atoi(env), kMaxSplitK64);
  } else {
    S = std::min(kMaxSplitK64, std::max(1, (num_cu + B - 1) / B));
    while (S > 1 && (V + S - 1) / S < 2048) S--;
  }
  return std::max(S, smin);
}

// Chunks per row: about four workgroups per CU, chunks of at least one
// 8192-id tile, at most kMaxSplit.  TGS_SPLIT overrides (tuning).
int choose_split(int num_cu, int ws_rows, int B, int V) {
  const int tile = 8192;
  int S = 1;
  const char* env = std::getenv("TGS_SPLIT");
  if (env && std::atoi(env) > 0) {
    S = std::min(std::atoi(env), kMaxSplit);
  } else {
    const int target = 4 * num_cu;
    while (S * 2 <= kMaxSplit && (long long)S * 2 * B <= target && (V + S * 2 - 1) / (S * 2) >= tile / 2) S *= 2;
  }
  while (S > 1 && (long long)S * B > ws_rows) S >>= 1;
  return S;
}

// Static LDS of the fused kernel beyond its dynamic carve-up (wave lists,
// staging, the radix-select scratch and the merge's words), with room for
// alignment.
size_t k64_static() { return tgs::k64_static_lds() + 256; }

// Whether a split k64 launch of `wgs` workgroups is resident on the device
// at once (then its chunks can wait on each other for the row-wide bound),
// from the runtime's occupancy of the instantiation; cached per variant and
// LDS size.  TGS_XCHG=0 turns the exchange off (tuning, tests).
bool k64_resident(int num_cu, int dt, bool whole_vec, bool mask, size_t lds, long long wgs) {
  const char* env = std::getenv("TGS_XCHG");
  if (env && std::atoi(env) == 0) return false;
  struct Entry {
    int key;
    size_t lds;
    int n;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  const int key = dt * 4 + (whole_vec ? 2 : 0) + (mask ? 1 : 0);
  int n = -1;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.key == key && e.lds == lds) n = e.n;
  }
  if (n < 0) {
    n = tgs::k64_resident_per_cu(dt, whole_vec, mask, lds);
    std::lock_guard<std::mutex> lock(mu);
    cache.push_back({key, lds, n});
  }
  return n > 0 && wgs <= (long long)n * num_cu;
}

// What a sampling call launches with: the device's size, and the workspace
// and mask table it uses (a handle's allocations, or the allocation-free
// entry point's static scratch and the caller's table).
struct SampleRes {
  int num_cu = 256;
  size_t lds_limit = 65536;
  unsigned long long* ws = nullptr;  // [ws_rows][KMAX] general-path chunk lists
  int* ws_cnt = nullptr;             // [ws_rows * (KMAX / 64)]
  int ws_rows = 0;
  unsigned* k64_cnt = nullptr;              // [rows * K64_CNT_STRIDE], zeroed at set-up
  unsigned long long* k64_lists = nullptr;  // [rows * kMaxSplit][64], entries 0 between calls
  unsigned long long* k64_keys = nullptr;   // [rows * K64_KEYS], zeroed at set-up
  const uint32_t* mask_table = nullptr;     // nullptr: no table
  int n_states = 0, mask_words = 0;
};

int efail(std::string& err, int code, const std::string& msg) {
  err = msg;
  return code;
}

// Validates the call and launches the kernels the batch hint selects (the
// body of tgs_sample, shared with tgs_sample_noalloc).  The device must be
// current; B, V and hist_cap must be within what res was sized for.
int sample_core(const SampleRes& res, std::string& err, const void* d_logits, tgs_dtype dt, int B, int V,
                int64_t row_stride, const int32_t* d_hist, const int32_t* d_hist_len, int hist_cap,
                const tgs_row_params* d_params, const float* d_u, int32_t* d_out_ids, const tgs_batch_hint* hint,
                const tgs_debug* dbg, hipStream_t stream) {
  if (dt != TGS_F32 && dt != TGS_BF16) return efail(err, TGS_EINVAL, "dtype");
  if (B < 0 || V < 1 || row_stride < V) return efail(err, TGS_EINVAL, "shape");
  if (B == 0) return TGS_OK;
  if (hist_cap < 0 || (hist_cap > 0 && !d_hist)) return efail(err, TGS_EINVAL, "history");
  if (!d_logits || !d_params || !d_u || !d_out_ids) return efail(err, TGS_EINVAL, "null buffer");
  tgs_debug dz;
  std::memset(&dz, 0, sizeof(dz));
  if (dbg) {
    dz = *dbg;
    if (dz.kept_cap < 0 || ((dz.kept_ids || dz.kept_probs) && dz.kept_cap == 0))
      return efail(err, TGS_EINVAL, "debug kept_cap");
  }
  const size_t esz = dt == TGS_BF16 ? 2 : 4;
  tgs::SampleArgs a;
  std::memset(&a, 0, sizeof(a));
  a.logits = d_logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.aligned = ((uintptr_t)d_logits % 16 == 0) && (((uint64_t)row_stride * esz) % 16 == 0);
  a.whole_vec = a.aligned && ((uint64_t)V * esz) % 16 == 0;
  a.hist = d_hist;
  a.hist_len = d_hist_len;
  a.hist_cap = hist_cap;
  a.params = d_params;
  a.u = d_u;
  a.out = d_out_ids;
  a.mask_table = res.mask_table;
  a.n_states = res.mask_table ? res.n_states : 0;
  a.mask_words = res.mask_words;
  a.ws = res.ws;
  a.ws_cnt = res.ws_cnt;
  a.cnt = res.k64_cnt;
  a.lists = res.k64_lists;
  a.keys = res.k64_keys;
  a.dbg = dz;
  // Kernels: the fused top_k <= 64 kernel when the hint says every row is
  // greedy or has top_k <= 64; otherwise the chunk kernel (+ merge kernel
  // for split rows), plus the full-path kernel when the hint allows rows
  // without a usable top-k.
  const int mk = hint ? hint->max_top_k : 0x7FFFFFFF;
  a.hint_k = mk;
  a.TS = hist_cap > 0 ? next_pow2(std::max(64, 2 * hist_cap)) : 0;
  a.ts_shift = a.TS ? 32 - log2i(a.TS) : 0;
  if (mk <= 64 && mk < V && hist_cap <= tgs::K64_MAX_HIST) {
    a.full_rows = 0;
    const int S = choose_split_k64(res.num_cu, B, V, dt);
    const int epv = dt == TGS_BF16 ? 8 : 4;
    const int L = ((V + S - 1) / S + epv - 1) / epv * epv;  // whole vectors: chunk starts stay aligned
    a.S = (V + L - 1) / L;
    a.L = L;
    // dynamic LDS: history hash, history bits of the chunk (packed per
    // thread: one bit per id of the largest chunk), candidate buffer (+16
    // pad entries for the ranking)
    a.BW = tgs::k64_chunk_ids(dt) / 32;
    a.off_hash = 0;
    a.off_bitmap = a.TS * 8;
    a.off_cand = (a.off_bitmap + a.BW * 4 + 15) / 16 * 16;
    a.capt = tgs::K64_CAP;
    a.ws_stride = 64;
    const size_t lds = (size_t)a.off_cand + (size_t)(tgs::K64_CAP + 16) * 8;
    if (lds + k64_static() > res.lds_limit) return efail(err, TGS_ETOOBIG, "history / vocab too large for LDS");
    if (a.S > 1 && V > (1 << 18)) return efail(err, TGS_ETOOBIG, "vocab beyond 2^18 ids (split-row list entries)");
    // split rows share a row-wide bound when every workgroup of the launch
    // is resident at once: each wave publishes its kq largest thread maxima
    // (at least 64 keys per row, at most K64_KEYS)
    a.xchg = a.S > 1 && k64_resident(res.num_cu, dt, a.whole_vec != 0, res.mask_table != nullptr && res.n_states > 0,
                                     lds, (long long)B * a.S);
    // keys per wave: the row's S * waves * kq keys fit its K64_KEYS slots
    a.kq = a.S >= 4 ? 4 : 8;
    while (a.kq > 1 && a.S * (tgs::K64_NT / 64) * a.kq > tgs::K64_KEYS) a.kq /= 2;
    // polls of the row's keys before a chunk keeps its own bound: far more
    // than a resident row needs (TGS_KEY_SPINS overrides: tests)
    {
      const char* env = std::getenv("TGS_KEY_SPINS");
      a.key_spins = env ? std::max(0, std::atoi(env)) : 2048;
    }
    // polls of the row's lists before the merging workgroup gives up and
    // writes id -4 (TGS_MERGE_SPINS overrides: tests force the give-up)
    {
      const char* env = std::getenv("TGS_MERGE_SPINS");
      a.merge_spins = env ? std::max(0, std::atoi(env)) : (1 << 18);
    }
    // the chunks of a row on one XCD (workgroups are dealt out to the XCDs in
    // turn); TGS_XMAP=0 turns it off
    {
      const char* env = std::getenv("TGS_XMAP");
      a.xmap = a.S > 1 && B % 8 == 0 && !(env && std::atoi(env) == 0);
    }
    // a row in one chunk that one wave holds: the one-wave variant (its
    // barriers and merges involve a single wave)
    const bool small = a.S == 1 && V <= tgs::k64_small_ids(dt) && hist_cap <= tgs::K64_SMALL_MAX_HIST;
    if (std::getenv("TGS_LOG_LAUNCH"))  // diagnostics: the launch's shape
      std::fprintf(stderr, "tgs k64: B=%d V=%d S=%d L=%d lds=%zu xchg=%d kq=%d xmap=%d small=%d\n", B, V, a.S, a.L,
                   lds, a.xchg, a.kq, a.xmap, (int)small);
    hipError_t e = tgs::launch_k64(a, dt, lds, stream, small);
    if (e != hipSuccess) return efail(err, TGS_EHIP, std::string("sample kernel launch: ") + hipGetErrorString(e));
    return TGS_OK;
  }
  if (mk <= tgs::KMAX && mk < V && V <= tgs::topk_max_vocab(dt) && a.whole_vec && hist_cap <= tgs::KMAX &&
      tgs::topk_lds_bytes(V, a.TS) + 2 * sizeof(tgs::BlockScratch) <= res.lds_limit) {
    // every row greedy or 1 <= top_k <= KMAX, the row fits in registers: one
    // workgroup per row
    a.full_rows = 0;
    a.S = 1;
    a.L = V;
    hipError_t e = tgs::launch_topk(a, dt, tgs::topk_lds_bytes(V, a.TS), stream);
    if (e != hipSuccess) return efail(err, TGS_EHIP, std::string("sample kernel launch: ") + hipGetErrorString(e));
    return TGS_OK;
  }
  const int mink = hint ? hint->min_top_k : 0;
  if (mk >= V && mink >= V && tgs::topp_lds_bytes(V, a.TS) + 2 * sizeof(tgs::BlockScratch) <= res.lds_limit) {
    // every sampling row without a usable top-k: the top-p kernel serves the
    // batch alone, greedy rows included (one workgroup per row)
    a.full_rows = 1;
    a.topp_all = 1;
    a.S = 1;
    a.L = V;
    a.topp_cap = tgs::topp_pack_cap(V, a.TS, res.lds_limit - 2 * sizeof(tgs::BlockScratch));
    hipError_t e = tgs::launch_topp(a, dt, stream);
    if (e != hipSuccess) return efail(err, TGS_EHIP, std::string("sample kernel launch: ") + hipGetErrorString(e));
    return TGS_OK;
  }
  a.full_rows = (mk > tgs::KMAX || mk >= V) ? 1 : 0;
  const int S = choose_split(res.num_cu, res.ws_rows, B, V);
  const int L = S > 1 ? ((V + S - 1) / S + 1023) / 1024 * 1024 : V;
  a.ws_stride = tgs::KMAX;
  a.S = (V + L - 1) / L;
  a.L = L;
  a.BW = hist_cap > 0 ? (L + 31) / 32 : 0;
  a.capt = tgs::CAPB + hist_cap;
  a.off_hash = 0;
  a.off_bitmap = a.TS * 8;
  a.off_cand = (a.off_bitmap + a.BW * 4 + 15) / 16 * 16;
  const size_t lds = (size_t)a.off_cand + (size_t)a.capt * 8;
  if (lds + sizeof(tgs::BlockScratch) > res.lds_limit)
    return efail(err, TGS_ETOOBIG, "history / vocab too large for LDS");
  if (a.full_rows && tgs::topp_lds_bytes(V, a.TS) + 2 * sizeof(tgs::BlockScratch) > res.lds_limit)
    return efail(err, TGS_ETOOBIG, "history / vocab too large for LDS (top-p rows)");
  a.topp_cap = tgs::topp_pack_cap(V, a.TS, res.lds_limit - 2 * sizeof(tgs::BlockScratch));
  hipError_t e = tgs::launch_sample(a, dt, lds, stream);
  if (e != hipSuccess) return efail(err, TGS_EHIP, std::string("sample kernel launch: ") + hipGetErrorString(e));
  return TGS_OK;
}

// ---------------------------------------------------------------- allocation-free sampling
//
// tgs_sample_noalloc takes its workspace from `scratch`, a static device
// array of fixed size (each GPU the library runs on holds its own copy until
// the process ends) instead of a handle's allocations:
//   [k64 chunk lists: kNaRows * kMaxSplit * 64 u64, entries 0 between calls]
//   [k64 bound-exchange keys: kNaRows * K64_KEYS u64]
//   [general-path chunk lists: kNaWsRows * KMAX u64]
//   [k64 exchange lines: kNaRows * K64_CNT_STRIDE u32, counters zero between calls]
//   [general-path list counts: kNaWsRows * (KMAX / 64) i32]
// The k64 kernel leaves its lists and counters in that state after every
// call; the first call on a device zeroes the whole array with a fill kernel
// (a call with B = 0 does only that, outside any graph capture).
// Host code never passes `scratch` itself to a kernel: its address on each
// device comes from hipGetSymbolAddress.
constexpr int kNaRows = 256;    // rows per call
constexpr int kNaWsRows = 512;  // general-path (row, chunk) lists
constexpr int kNaHist = tgs::K64_MAX_HIST;
constexpr size_t kNaListWords = (size_t)kNaRows * kMaxSplitK64 * 64;
constexpr size_t kNaKeyWords = (size_t)kNaRows * tgs::K64_KEYS;
constexpr size_t kNaWsWords = (size_t)kNaWsRows * tgs::KMAX;
constexpr size_t kNaCntU32 = (size_t)kNaRows * tgs::K64_CNT_STRIDE;
constexpr size_t kNaWsCntI32 = (size_t)kNaWsRows * (tgs::KMAX / 64);
constexpr size_t kNaWords = kNaListWords + kNaKeyWords + kNaWsWords + (kNaCntU32 + kNaWsCntI32) / 2;
static_assert(kNaCntU32 % 2 == 0 && kNaWsCntI32 % 2 == 0, "whole 8-byte words");

constexpr int kNaMaxDevices = 64;
struct NoAllocDevice {
  bool ready = false;
  unsigned long long* ptr = nullptr;  // this device's copy of scratch
  int num_cu = 256;
  size_t lds_limit = 65536;
};
std::mutex g_na_mu;
NoAllocDevice g_na[kNaMaxDevices];
thread_local std::string g_na_err;

__global__ void na_fill_kernel(unsigned long long* p, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0ull;
}

}  // namespace

static __device__ __align__(256) unsigned long long scratch[kNaWords];

namespace {

bool noalloc_ready(int device) {
  std::lock_guard<std::mutex> lock(g_na_mu);
  return g_na[device].ready;
}

// Once per device, with that device current: the address of its scratch,
// its size limits, the kernels' LDS ceilings and the lists' initial state.
int noalloc_setup(int device, NoAllocDevice*& out) {
  std::lock_guard<std::mutex> lock(g_na_mu);
  NoAllocDevice& d = g_na[device];
  if (!d.ready) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return efail(g_na_err, TGS_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    d.ptr = (unsigned long long*)ptr;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && v > 0)
      d.num_cu = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
      d.lds_limit = (size_t)v;
    if (tgs::set_sample_lds_limit(d.lds_limit - sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_k64_lds_limit(d.lds_limit - k64_static()) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_topp_lds_limit(d.lds_limit - 2 * sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_topk_lds_limit(d.lds_limit - 2 * sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    // everything zero: k64 lists "not written", counters and epochs zero
    hipLaunchKernelGGL(na_fill_kernel, dim3(1024), dim3(256), 0, nullptr, d.ptr, kNaWords);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return efail(g_na_err, TGS_EHIP, std::string("scratch set-up: ") + hipGetErrorString(e));
    d.ready = true;
  }
  out = &d;
  return TGS_OK;
}

}  // namespace

extern "C" {

int tgs_abi_version(void) { return TGS_ABI_VERSION; }

const char* tgs_status_string(int status) {
  switch (status) {
    case TGS_OK: return "ok";
    case TGS_EINVAL: return "invalid argument";
    case TGS_ENOMEM: return "device allocation failed";
    case TGS_EHIP: return "HIP runtime error";
    case TGS_EALLMASKED: return "no allowed token in the row";
    case TGS_ETOOBIG: return "size exceeds the handle's limits";
    default: return "unknown status";
  }
}

int tgs_hint_from_params(const tgs_row_params* p, int B, int V, tgs_batch_hint* out) {
  if (!out || B < 0 || V < 1 || (B > 0 && !p)) return TGS_EINVAL;
  int mk = 0, mn = V;
  for (int b = 0; b < B; b++) {
    const float T = p[b].temperature;
    const bool greedy = (p[b].flags & TGS_FLAG_GREEDY) || !(T > 0.0f);
    if (greedy) continue;
    const int k = (p[b].top_k >= 1 && p[b].top_k < V) ? p[b].top_k : V;
    mk = std::max(mk, k);
    mn = std::min(mn, k);
  }
  out->max_top_k = mk;
  out->min_top_k = mn;
  return TGS_OK;
}

int tgs_create(tgs_handle* out, int device, int max_batch, int max_vocab, int max_hist) {
  if (!out) return TGS_EINVAL;
  *out = nullptr;
  if (max_batch < 1 || max_vocab < 1 || max_vocab > kMaxVocab || max_hist < 0 || max_hist > kMaxHist)
    return TGS_EINVAL;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return TGS_EHIP;
  if (device < 0 || device >= ndev) return TGS_EINVAL;
  tgs_ctx* h = new (std::nothrow) tgs_ctx;
  if (!h) return TGS_ENOMEM;
  h->device = device;
  h->max_batch = max_batch;
  h->max_vocab = max_vocab;
  h->max_hist = max_hist;
  DeviceGuard g(device);
  if (!g.ok) {
    delete h;
    return TGS_EHIP;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && v > 0)
    h->num_cu = v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
    h->lds_limit = (size_t)v;
  h->ws_rows = std::max(max_batch, 4 * h->num_cu);
  hipError_t e = hipMalloc(&h->ws, sizeof(unsigned long long) * (size_t)h->ws_rows * tgs::KMAX);
  if (e == hipSuccess) e = hipMalloc(&h->ws_cnt, sizeof(int) * (size_t)h->ws_rows * (tgs::KMAX / 64));
  const size_t cnt_bytes = sizeof(unsigned) * (size_t)max_batch * tgs::K64_CNT_STRIDE;
  if (e == hipSuccess) e = hipMalloc(&h->k64_cnt, cnt_bytes);
  if (e == hipSuccess) e = hipMemset(h->k64_cnt, 0, cnt_bytes);
  const size_t list_bytes = sizeof(unsigned long long) * (size_t)max_batch * kMaxSplit * 64;
  if (e == hipSuccess) e = hipMalloc(&h->k64_lists, list_bytes);
  if (e == hipSuccess) e = hipMemset(h->k64_lists, 0, list_bytes);  // every entry "not written"
  const size_t key_bytes = sizeof(unsigned long long) * (size_t)max_batch * tgs::K64_KEYS;
  if (e == hipSuccess) e = hipMalloc(&h->k64_keys, key_bytes);
  if (e == hipSuccess) e = hipMemset(h->k64_keys, 0, key_bytes);
  if (e == hipSuccess) {
    // raise the dynamic-LDS ceiling to the device limit; a runtime that
    // rejects the attribute keeps its default (calls that need more fail
    // with TGS_ETOOBIG / TGS_EHIP instead)
    if (tgs::set_sample_lds_limit(h->lds_limit - sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_k64_lds_limit(h->lds_limit - k64_static()) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_topp_lds_limit(h->lds_limit - 2 * sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    if (tgs::set_topk_lds_limit(h->lds_limit - 2 * sizeof(tgs::BlockScratch)) != hipSuccess) (void)hipGetLastError();
    e = hipDeviceSynchronize();
  }
  if (e != hipSuccess) {
    tgs_destroy(h);
    return e == hipErrorOutOfMemory ? TGS_ENOMEM : TGS_EHIP;
  }
  *out = h;
  return TGS_OK;
}

void tgs_destroy(tgs_handle h) {
  if (!h) return;
  DeviceGuard g(h->device);
  if (h->ws) (void)hipFree(h->ws);
  if (h->ws_cnt) (void)hipFree(h->ws_cnt);
  if (h->k64_cnt) (void)hipFree(h->k64_cnt);
  if (h->k64_lists) (void)hipFree(h->k64_lists);
  if (h->k64_keys) (void)hipFree(h->k64_keys);
  if (h->mask_table) (void)hipFree(h->mask_table);
  if (h->mask_stage) (void)hipFree(h->mask_stage);
  free_spec(h);
  delete h;
}

const char* tgs_last_error(tgs_handle h) {
  if (h) return h->err.c_str();
  return g_na_err.empty() ? "null handle" : g_na_err.c_str();
}

int tgs_mask_table_set(tgs_handle h, const uint32_t* host_words, int n_states, int vocab) {
  if (!h) return TGS_EINVAL;
  if (n_states < 0 || vocab < 1 || (n_states > 0 && !host_words)) return fail(h, TGS_EINVAL, "mask table: bad arguments");
  DeviceGuard g(h->device);
  const int words = (vocab + 31) / 32;
  uint32_t* dptr = nullptr;
  const size_t bytes = sizeof(uint32_t) * (size_t)n_states * words;
  if (n_states > 0) {
    hipError_t e = hipMalloc(&dptr, bytes);
    if (e != hipSuccess) return fail(h, TGS_ENOMEM, "mask table allocation failed");
    e = hipMemcpy(dptr, host_words, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(dptr);
      return hip_fail(h, e, "mask table upload");
    }
  }
  if (h->mask_table) {
    (void)hipDeviceSynchronize();
    (void)hipFree(h->mask_table);
  }
  h->mask_table = dptr;
  h->n_states = n_states;
  h->mask_vocab = vocab;
  h->mask_words = words;
  return TGS_OK;
}

int tgs_mask_table_get(tgs_handle h, int first, int n, uint32_t* host_words) {
  if (!h) return TGS_EINVAL;
  if (first < 0 || n < 0 || first > h->n_states - n || (n > 0 && !host_words))
    return fail(h, TGS_EINVAL, "mask table get: rows outside the table");
  if (n == 0) return TGS_OK;
  DeviceGuard g(h->device);
  if (!g.ok) return fail(h, TGS_EHIP, "hipSetDevice");
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpy(host_words, h->mask_table + (size_t)first * h->mask_words,
                  sizeof(uint32_t) * (size_t)h->mask_words * (size_t)n, hipMemcpyDeviceToHost);
  return e == hipSuccess ? TGS_OK : hip_fail(h, e, "mask table readback");
}

int tgs_mask_table_update(tgs_handle h, const int32_t* host_states, const uint32_t* host_words, int n) {
  if (!h) return TGS_EINVAL;
  if (n < 0 || (n > 0 && (!host_states || !host_words))) return fail(h, TGS_EINVAL, "mask update: bad arguments");
  for (int i = 0; i < n; i++)
    if (host_states[i] < 0 || host_states[i] >= h->n_states) return fail(h, TGS_EINVAL, "mask update: state out of range");
  if (n == 0) return TGS_OK;
  DeviceGuard g(h->device);
  const size_t row_bytes = sizeof(uint32_t) * (size_t)h->mask_words;
  // consecutive states: one copy straight into the table
  bool run = true;
  for (int i = 1; i < n && run; i++) run = host_states[i] == host_states[0] + i;
  if (run) {
    hipError_t e = hipMemcpy(h->mask_table + (size_t)host_states[0] * h->mask_words, host_words, row_bytes * n,
                             hipMemcpyHostToDevice);
    return e == hipSuccess ? TGS_OK : hip_fail(h, e, "mask update upload");
  }
  // otherwise one upload of the rows (the last of repeated states wins) and
  // their destinations, then one scatter launch
  std::vector<int> last(n);
  {
    std::unordered_map<int, int> pos;
    for (int i = 0; i < n; i++) pos[host_states[i]] = i;
    int m = 0;
    for (int i = 0; i < n; i++)
      if (pos[host_states[i]] == i) last[m++] = i;
    last.resize(m);
  }
  const int m = (int)last.size();
  const size_t head = ((sizeof(int) * 2 * (size_t)m) + 255) / 256 * 256;
  const size_t need = head + row_bytes * n;
  if (need > h->mask_stage_bytes) {
    if (h->mask_stage) {
      (void)hipDeviceSynchronize();
      (void)hipFree(h->mask_stage);
      h->mask_stage = nullptr;
      h->mask_stage_bytes = 0;
    }
    if (hipMalloc(&h->mask_stage, need) != hipSuccess) return fail(h, TGS_ENOMEM, "mask update staging");
    h->mask_stage_bytes = need;
  }
  std::vector<char> up(need);
  int* packed = (int*)up.data();
  for (int r = 0; r < m; r++) {
    packed[r] = host_states[last[r]];
    packed[m + r] = last[r];
  }
  std::memcpy(up.data() + head, host_words, row_bytes * n);
  char* stage = (char*)h->mask_stage;
  hipError_t e = hipMemcpy(stage, up.data(), need, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(h, e, "mask update upload");
  e = tgs::launch_mask_scatter((const int*)stage, (const uint32_t*)(stage + head), m, h->mask_words, h->mask_table,
                               nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  return e == hipSuccess ? TGS_OK : hip_fail(h, e, "mask update scatter");
}

int tgs_sample(tgs_handle h, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
               const int32_t* d_hist, const int32_t* d_hist_len, int hist_cap,
               const tgs_row_params* d_params, const float* d_u, int32_t* d_out_ids,
               const tgs_batch_hint* hint, const tgs_debug* dbg, tgs_stream stream) {
  if (!h) return TGS_EINVAL;
  if (dt != TGS_F32 && dt != TGS_BF16) return fail(h, TGS_EINVAL, "dtype");
  if (B < 0 || V < 1 || row_stride < V) return fail(h, TGS_EINVAL, "shape");
  if (B == 0) return TGS_OK;
  if (B > h->max_batch || V > h->max_vocab || hist_cap > h->max_hist)
    return fail(h, TGS_ETOOBIG, "batch, vocab or history beyond the handle's limits");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(h, TGS_EHIP, "hipSetDevice");
  SampleRes res;
  res.num_cu = h->num_cu;
  res.lds_limit = h->lds_limit;
  res.ws = h->ws;
  res.ws_cnt = h->ws_cnt;
  res.ws_rows = h->ws_rows;
  res.k64_cnt = h->k64_cnt;
  res.k64_lists = h->k64_lists;
  res.k64_keys = h->k64_keys;
  const bool table_ok = h->mask_table && h->mask_vocab >= V;
  res.mask_table = table_ok ? h->mask_table : nullptr;
  res.n_states = table_ok ? h->n_states : 0;
  res.mask_words = h->mask_words;
  return sample_core(res, h->err, d_logits, dt, B, V, row_stride, d_hist, d_hist_len, hist_cap, d_params, d_u,
                     d_out_ids, hint, dbg, (hipStream_t)stream);
}

int tgs_sample_noalloc(int device, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
                       const int32_t* d_hist, const int32_t* d_hist_len, int hist_cap,
                       const tgs_row_params* d_params, const float* d_u, int32_t* d_out_ids,
                       const uint32_t* d_mask_table, int n_states, int mask_vocab, const tgs_batch_hint* hint,
                       const tgs_debug* dbg, tgs_stream stream) {
  if (dt != TGS_F32 && dt != TGS_BF16) return efail(g_na_err, TGS_EINVAL, "dtype");
  if (B < 0 || V < 1 || row_stride < V) return efail(g_na_err, TGS_EINVAL, "shape");
  if (B > kNaRows || V > kMaxVocab || hist_cap > kNaHist)
    return efail(g_na_err, TGS_ETOOBIG,
                 "tgs_sample_noalloc: at most " + std::to_string(kNaRows) + " rows, " + std::to_string(kMaxVocab) +
                     " ids per row and " + std::to_string(kNaHist) + " history ids per row (its static workspace)");
  if (n_states < 0 || (n_states > 0 && (!d_mask_table || mask_vocab < V)))
    return efail(g_na_err, TGS_EINVAL, "mask table: n_states >= 0; a table needs a pointer and mask_vocab >= V");
  if (device < 0 || device >= kNaMaxDevices) return efail(g_na_err, TGS_EINVAL, "device");
  DeviceGuard g(device);
  if (!g.ok) return efail(g_na_err, TGS_EHIP, "hipSetDevice");
  // The device's set-up (a fill kernel and a synchronisation) cannot run
  // under graph capture: the first call on a device, which a call with B = 0
  // can be, has to come before any capture.
  NoAllocDevice* d = nullptr;
  if (!noalloc_ready(device)) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return efail(g_na_err, TGS_EINVAL,
                   "tgs_sample_noalloc: the first call on a device sets it up and must not be captured "
                   "(call it once with B = 0 before capturing)");
  }
  const int rc = noalloc_setup(device, d);
  if (rc != TGS_OK) return rc;
  if (B == 0) return TGS_OK;
  SampleRes res;
  res.num_cu = d->num_cu;
  res.lds_limit = d->lds_limit;
  res.k64_lists = d->ptr;
  res.k64_keys = d->ptr + kNaListWords;
  res.ws = d->ptr + kNaListWords + kNaKeyWords;
  res.ws_rows = kNaWsRows;
  res.k64_cnt = (unsigned*)(d->ptr + kNaListWords + kNaKeyWords + kNaWsWords);
  res.ws_cnt = (int*)(res.k64_cnt + kNaCntU32);
  res.mask_table = n_states > 0 ? d_mask_table : nullptr;
  res.n_states = n_states;
  res.mask_words = (mask_vocab + 31) / 32;
  return sample_core(res, g_na_err, d_logits, dt, B, V, row_stride, d_hist, d_hist_len, hist_cap, d_params, d_u,
                     d_out_ids, hint, dbg, (hipStream_t)stream);
}

int tgs_mask_rows_from_dfa(tgs_handle h, const uint8_t* d_byte_class, const int32_t* d_trans, int n_cls,
                           const uint8_t* d_complete, int n_dfa, const int32_t* d_tok_off,
                           const uint8_t* d_tok_bytes, int64_t n_bytes, int n_tokens, int eos_id,
                           const int32_t* d_states, const int32_t* d_rows, int n, tgs_stream stream) {
  if (!h) return TGS_EINVAL;
  if (n < 0 || n_dfa < 1 || n_cls < 1 || n_cls > 256 || n_tokens < 0 || eos_id < -1 || eos_id >= n_tokens ||
      n_bytes < 0)
    return fail(h, TGS_EINVAL, "mask build: bad arguments");
  if (n == 0) return TGS_OK;
  if (!d_byte_class || !d_trans || !d_complete || !d_tok_off || (!d_tok_bytes && n_bytes > 0) || !d_states ||
      !d_rows)
    return fail(h, TGS_EINVAL, "null buffer");
  if (!h->mask_table || h->n_states < 1) return fail(h, TGS_EINVAL, "mask build: no mask table (tgs_mask_table_set)");
  if (n_tokens > h->mask_vocab) return fail(h, TGS_ETOOBIG, "mask build: more tokens than the table's vocabulary");
  if (n > tgs::MASK_SPW_LDS * 65535) return fail(h, TGS_ETOOBIG, "mask build: at most 1048560 rows per call");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(h, TGS_EHIP, "hipSetDevice");
  tgs::MaskBuildArgs a;
  std::memset(&a, 0, sizeof(a));
  a.byte_class = d_byte_class;
  a.trans = d_trans;
  a.n_cls = n_cls;
  a.complete = d_complete;
  a.n_dfa = n_dfa;
  // LDS path: the 16-bit table fits LDS (and its offsets 16 bits) and its image fits the
  // handle's workspace, where it is prepared once per call (calls on one handle are ordered
  // on one stream)
  const size_t ws_bytes = sizeof(unsigned long long) * (size_t)h->ws_rows * tgs::KMAX;
  a.lds = tgs::mask_lds_table_bytes(n_dfa, n_cls) <= (size_t)tgs::MASK_LDS_TABLE &&
          tgs::mask_image_bytes(n_dfa, n_cls) <= ws_bytes;
  a.image = (uint16_t*)h->ws;
  a.tok_off = d_tok_off;
  a.tok_bytes = d_tok_bytes;
  // offsets are int32: no token can end past INT32_MAX bytes
  a.n_bytes = n_bytes < (int64_t)INT32_MAX ? (int)n_bytes : INT32_MAX;
  a.n_tokens = n_tokens;
  a.eos = eos_id;
  a.states = d_states;
  a.rows = d_rows;
  a.n = n;
  a.table = h->mask_table;
  a.n_rows = h->n_states;
  a.words = h->mask_words;
  hipError_t e = tgs::launch_mask_build(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(h, e, "mask build launch");
  return TGS_OK;
}

int tgs_token_logprobs(tgs_handle h, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
                       const int32_t* d_tokens, float* d_out_logprob, float* d_out_lse, tgs_stream stream) {
  if (!h) return TGS_EINVAL;
  if (dt != TGS_F32 && dt != TGS_BF16) return fail(h, TGS_EINVAL, "dtype");
  if (B < 0 || V < 1 || row_stride < V) return fail(h, TGS_EINVAL, "shape");
  if (B == 0) return TGS_OK;
  if (!d_logits || !d_tokens || !d_out_logprob) return fail(h, TGS_EINVAL, "null buffer");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(h, TGS_EHIP, "hipSetDevice");
  const size_t esz = dt == TGS_BF16 ? 2 : 4;
  const int epv = dt == TGS_BF16 ? 8 : 4;
  tgs::LogprobArgs a;
  std::memset(&a, 0, sizeof(a));
  a.logits = d_logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.aligned = ((uintptr_t)d_logits % 16 == 0) && (((uint64_t)row_stride * esz) % 16 == 0);
  a.tokens = d_tokens;
  a.out_lp = d_out_logprob;
  a.out_lse = d_out_lse;
  // enough workgroups for the chip: short batches split rows into chunks of
  // at least 4096 ids (whole vectors) whose partial sums a second launch
  // combines through the handle's workspace
  const int target = 4 * h->num_cu;
  int S = B >= target ? 1 : (target + B - 1) / B;
  S = std::min(S, (V + 4095) / 4096);
  S = std::max(S, 1);
  const size_t ws_floats = (size_t)h->ws_rows * tgs::KMAX * 2;
  if ((size_t)B * S * 2 > ws_floats) S = 1;
  int L = (V + S - 1) / S;
  L = (L + epv - 1) / epv * epv;
  a.S = (V + L - 1) / L;
  a.L = L;
  a.part = (float*)h->ws;
  hipError_t e = tgs::launch_logprob(a, dt == TGS_BF16 ? 1 : 0, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(h, e, "logprob kernel launch");
  return TGS_OK;
}

int tgs_reserve_spec(tgs_handle h, int max_batch, int max_k) {
  if (!h) return TGS_EINVAL;
  if (max_batch < 1 || max_k < 0 || max_k > 64) return fail(h, TGS_EINVAL, "spec reserve");
  if (max_batch <= h->spec_b && max_k <= h->spec_k) return TGS_OK;
  DeviceGuard g(h->device);
  (void)hipDeviceSynchronize();
  const int nb = std::max(max_batch, h->spec_b);
  const int nk = std::max(max_k, h->spec_k);
  free_spec(h);
  // per row: block maxima and masses for every block of the handle's vocab
  const size_t rows = (size_t)nb * (2 * nk + 1);
  const int nbs = (h->max_vocab + tgs::SPEC_BLOCK - 1) / tgs::SPEC_BLOCK;
  hipError_t e = hipMalloc(&h->spec_blk_m, sizeof(float) * rows * nbs);
  if (e == hipSuccess) e = hipMalloc(&h->spec_blk_q, sizeof(unsigned long long) * rows * nbs);
  if (e == hipSuccess) e = hipMalloc(&h->spec_blk_w, sizeof(unsigned long long) * (size_t)nb * nbs * tgs::SPEC_GROUPS);
  if (e == hipSuccess) e = hipMalloc(&h->spec_state, (size_t)32 * nb);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    free_spec(h);
    return fail(h, TGS_ENOMEM, "spec workspace allocation failed");
  }
  h->spec_b = nb;
  h->spec_k = nk;
  h->spec_nbs = nbs;
  return TGS_OK;
}

int tgs_spec_verify(tgs_handle h, const void* d_target, const void* d_draft, tgs_dtype dt,
                    const int32_t* d_draft_tok, int B, int k, int V, const float* d_T,
                    const float* d_u_acc, const float* d_u_res, int32_t* d_n_acc, int32_t* d_out,
                    tgs_stream stream) {
  if (!h) return TGS_EINVAL;
  if (dt != TGS_F32 && dt != TGS_BF16) return fail(h, TGS_EINVAL, "dtype");
  if (B < 0 || k < 0 || k > 64 || V < 1) return fail(h, TGS_EINVAL, "shape");
  if (B == 0) return TGS_OK;
  if (V > h->max_vocab) return fail(h, TGS_ETOOBIG, "vocab beyond the handle's limit");
  if (!d_target || (k > 0 && (!d_draft || !d_draft_tok || !d_u_acc)) || !d_T || !d_u_res || !d_n_acc || !d_out)
    return fail(h, TGS_EINVAL, "null buffer");
  if (B > h->spec_b || k > h->spec_k) {
    int rc = tgs_reserve_spec(h, B, k);
    if (rc != TGS_OK) return rc;
  }
  DeviceGuard g(h->device);
  if (!g.ok) return fail(h, TGS_EHIP, "hipSetDevice");
  const size_t esz = dt == TGS_BF16 ? 2 : 4;
  tgs::SpecArgs a;
  std::memset(&a, 0, sizeof(a));
  a.target = d_target;
  a.draft = d_draft;
  a.B = B;
  a.k = k;
  a.V = V;
  a.aligned = ((uintptr_t)d_target % 16 == 0) && ((uintptr_t)d_draft % 16 == 0) && (((uint64_t)V * esz) % 16 == 0);
  a.dtok = d_draft_tok;
  a.T = d_T;
  a.u_acc = d_u_acc;
  a.u_res = d_u_res;
  a.n_acc = d_n_acc;
  a.out = d_out;
  a.nb = (V + tgs::SPEC_BLOCK - 1) / tgs::SPEC_BLOCK;
  a.nbs = h->spec_nbs;
  a.blk_m = h->spec_blk_m;
  a.blk_q = h->spec_blk_q;
  a.blk_w = h->spec_blk_w;
  a.seq_state = h->spec_state;
  a.ncu = h->num_cu;
  hipError_t e = tgs::launch_spec(a, dt, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(h, e, "spec kernel launch");
  return TGS_OK;
}

}  // extern "C"
