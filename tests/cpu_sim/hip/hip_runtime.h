// hip_runtime.h (CPU simulation) -- runs the sampler's HIP kernels on host
// threads so that their memory accesses can be checked with AddressSanitizer
// and debugged with gdb.  TEST INFRASTRUCTURE ONLY, never part of the product.
//
// Model: a launch runs its blocks one after another; a block is blockDim.x
// OS threads.  __syncthreads is a barrier over the block's threads; wave
// intrinsics (__shfl*, __ballot) exchange values among the 64 threads of a
// wave through a per-wave buffer between two barriers.  A thread leaving
// the kernel drops out of its barriers (exited waves do not take part in
// later barriers on the GPU either).  __shared__ variables are static (one
// instance per kernel); a kernel whose static LDS is one TGS_STATIC_SMEM
// object gets a copy per block instead.  With TGS_SIM_CONCURRENT set, every
// block of a launch runs at once (for kernels whose blocks wait on each
// other; only kernels with no plain __shared__ variables may run so).
// Device memory is host memory.
#pragma once

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <thread>
#include <type_traits>
#include <vector>

#include <linux/futex.h>
#include <sys/syscall.h>
#include <unistd.h>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __noinline__ __attribute__((noinline))
#define __launch_bounds__(...)
// Static LDS variables live in one linker section so that every block can
// start with it poisoned (LDS holds garbage at kernel start on the GPU).
#define __shared__ static __attribute__((section("tgs_lds")))
extern "C" unsigned char __start_tgs_lds[], __stop_tgs_lds[];
#define __align__(x) alignas(x)
#define TGS_DYN_SMEM(name) unsigned char* name = hipcpu::dyn_smem()
#define TGS_STATIC_SMEM(type, name) type& name = *reinterpret_cast<type*>(hipcpu::static_smem(sizeof(type)))

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint4 {
  uint32_t x, y, z, w;
};
struct uint2 {
  uint32_t x, y;
};
struct int2 {
  int x, y;
};
static inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return {a, b, c, d}; }
static inline int2 make_int2(int a, int b) { return {a, b}; }

typedef int hipError_t;
typedef struct ihipStream_t* hipStream_t;
enum {
  hipSuccess = 0,
  hipErrorOutOfMemory = 2,
  hipErrorInvalidValue = 1,
  hipStreamCaptureStatusNone = 0,
  hipStreamCaptureStatusActive = 1,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipDeviceAttributeMultiprocessorCount = 1,
  hipDeviceAttributeMaxSharedMemoryPerBlock = 2,
  hipFuncAttributeMaxDynamicSharedMemorySize = 3,
};

namespace hipcpu {

// A reusable barrier over n threads, with arrive_and_drop for a thread that
// leaves.  Arrivals count down one word; the last arrival resets the count,
// advances the generation word and wakes every waiter with one futex call,
// and a waiter sleeps on the generation word until it moves (no mutex, so the
// woken threads do not queue for a lock; GCC 11's std::barrier hung now and
// then here when threads dropped out while others waited).  A thread reads
// the generation before it arrives: the generation cannot move before its own
// arrival, and a futex wait on a stale value returns at once.
class Barrier {
 public:
  explicit Barrier(unsigned n) : expected_(n), count_(n) {}
  void arrive_and_wait() {
    const uint32_t g = __atomic_load_n(&gen_, __ATOMIC_ACQUIRE);
    if (__atomic_sub_fetch(&count_, 1u, __ATOMIC_ACQ_REL) == 0) {
      next_phase();
      return;
    }
    while (__atomic_load_n(&gen_, __ATOMIC_ACQUIRE) == g)
      syscall(SYS_futex, &gen_, FUTEX_WAIT_PRIVATE, g, nullptr, nullptr, 0);
  }
  void arrive_and_drop() {
    // the expected count drops before this arrival counts, so the arrival
    // that completes the phase reads it
    __atomic_sub_fetch(&expected_, 1u, __ATOMIC_ACQ_REL);
    if (__atomic_sub_fetch(&count_, 1u, __ATOMIC_ACQ_REL) == 0) next_phase();
  }

 private:
  void next_phase() {
    __atomic_store_n(&count_, __atomic_load_n(&expected_, __ATOMIC_ACQUIRE), __ATOMIC_RELAXED);
    __atomic_add_fetch(&gen_, 1u, __ATOMIC_RELEASE);
    syscall(SYS_futex, &gen_, FUTEX_WAKE_PRIVATE, INT32_MAX, nullptr, nullptr, 0);
  }
  uint32_t expected_, count_;
  uint32_t gen_ = 0;
};

struct WaveCtx {
  std::unique_ptr<Barrier> bar;
  uint64_t buf[64];
};
constexpr size_t kStaticSmem = 65536;  // per-block static LDS object (TGS_STATIC_SMEM) at most
struct BlockCtx {
  std::unique_ptr<Barrier> bar;
  std::vector<WaveCtx> waves;
  std::vector<unsigned char> smem;
  std::vector<unsigned char> ssmem;
};
inline thread_local BlockCtx* t_ctx = nullptr;
inline BlockCtx*& block_ctx() { return t_ctx; }
inline thread_local dim3 t_thread, t_block;
inline dim3 g_block_dim, g_grid_dim;
inline unsigned char* dyn_smem() { return block_ctx()->smem.data(); }
inline unsigned char* static_smem(size_t n) {
  if (n > kStaticSmem) std::abort();
  return block_ctx()->ssmem.data();
}

inline int lane() { return (int)(t_thread.x & 63); }
inline WaveCtx& wave() { return block_ctx()->waves[t_thread.x / 64]; }

template <typename T>
inline uint64_t to_bits(T x) {
  uint64_t u = 0;
  std::memcpy(&u, &x, sizeof(T));
  return u;
}
template <typename T>
inline T from_bits(uint64_t u) {
  T x;
  std::memcpy(&x, &u, sizeof(T));
  return x;
}
template <typename T>
inline T exchange(T x, int src) {
  WaveCtx& w = wave();
  w.buf[lane()] = to_bits(x);
  w.bar->arrive_and_wait();
  const uint64_t r = (src >= 0 && src < 64) ? w.buf[src] : w.buf[lane()];
  w.bar->arrive_and_wait();
  return from_bits<T>(r);
}

template <typename... Args>
inline void launch(void (*k)(Args...), dim3 grid, dim3 block, size_t shmem, Args... args) {
  g_grid_dim = grid;
  g_block_dim = block;
  if (std::getenv("TGS_SIM_TRACE"))  // launch log (tests check which kernel ran)
    std::fprintf(stderr, "launch grid=%u block=%u lds=%zu\n", grid.x, block.x, shmem);
  const unsigned nt = block.x;
  const unsigned nblk = grid.x * grid.y;
  const bool conc = std::getenv("TGS_SIM_CONCURRENT") != nullptr;
  // blocks started together (a launch too large to run as threads at once,
  // such as a set-up fill over a whole workspace, runs block by block)
  const unsigned group = conc && (size_t)nblk * nt <= 16384 ? nblk : 1u;
  auto make_ctx = [&]() {
    auto ctx = std::make_unique<BlockCtx>();
    ctx->bar = std::make_unique<Barrier>(nt);
    ctx->waves.resize((nt + 63) / 64);
    for (unsigned w = 0; w < ctx->waves.size(); w++) {
      const unsigned n = std::min(64u, nt - 64 * w);
      ctx->waves[w].bar = std::make_unique<Barrier>(n);
    }
    ctx->smem.assign(shmem ? shmem : 1, 0xA5);
    ctx->ssmem.assign(kStaticSmem, 0xA5);
    return ctx;
  };
  auto run_thread = [=](BlockCtx* ctx, unsigned t, unsigned bi) {
    t_ctx = ctx;
    t_thread = dim3(t);
    t_block = dim3(bi % grid.x, bi / grid.x);
    k(args...);
    ctx->waves[t / 64].bar->arrive_and_drop();
    ctx->bar->arrive_and_drop();
  };
  if (group == 1) {
    // block by block on one set of nt threads (creating threads costs more
    // than the kernels here): the host thread sets each block up, a gate
    // lets the threads into it, and a second gate waits for all of them
    std::unique_ptr<BlockCtx> cur;
    Barrier gate(nt + 1);
    std::vector<std::thread> th;
    th.reserve(nt);
    for (unsigned t = 0; t < nt; t++)
      th.emplace_back([&, t]() {
        for (unsigned bi = 0; bi < nblk; bi++) {
          gate.arrive_and_wait();
          run_thread(cur.get(), t, bi);
          gate.arrive_and_wait();
        }
      });
    for (unsigned bi = 0; bi < nblk; bi++) {
      cur = make_ctx();
      std::memset(__start_tgs_lds, 0xA5, (size_t)(__stop_tgs_lds - __start_tgs_lds));
      gate.arrive_and_wait();
      gate.arrive_and_wait();
    }
    for (auto& x : th) x.join();
    return;
  }
  for (unsigned b0 = 0; b0 < nblk; b0 += group) {
    const unsigned nb = std::min(group, nblk - b0);
    std::vector<std::unique_ptr<BlockCtx>> ctxs(nb);
    for (unsigned i = 0; i < nb; i++) ctxs[i] = make_ctx();
    std::memset(__start_tgs_lds, 0xA5, (size_t)(__stop_tgs_lds - __start_tgs_lds));
    std::vector<std::thread> th;
    th.reserve((size_t)nb * nt);
    for (unsigned i = 0; i < nb; i++) {
      BlockCtx* ctx = ctxs[i].get();
      for (unsigned t = 0; t < nt; t++) th.emplace_back([=]() { run_thread(ctx, t, b0 + i); });
    }
    for (auto& x : th) x.join();
  }
}

}  // namespace hipcpu

#define threadIdx (hipcpu::t_thread)
#define blockIdx (hipcpu::t_block)
#define blockDim (hipcpu::g_block_dim)
#define gridDim (hipcpu::g_grid_dim)

#define hipLaunchKernelGGL(k, g, b, sh, st, ...) hipcpu::launch(k, dim3(g), dim3(b), (size_t)(sh), __VA_ARGS__)

inline void __syncthreads() { hipcpu::block_ctx()->bar->arrive_and_wait(); }
inline int __syncthreads_or(int pred) {
  static std::atomic<int> acc{0};
  __syncthreads();
  if (pred) acc.store(1);
  __syncthreads();
  const int r = acc.load();
  __syncthreads();
  if (threadIdx.x == 0) acc.store(0);
  __syncthreads();
  return r;
}
inline int __lane_id() { return hipcpu::lane(); }

template <typename T>
inline T __shfl(T x, int src, int width = 64) { (void)width; return hipcpu::exchange(x, src); }
template <typename T>
inline T __shfl_xor(T x, int m, int width = 64) { (void)width; return hipcpu::exchange(x, hipcpu::lane() ^ m); }
template <typename T>
inline T __shfl_up(T x, int d, int width = 64) {
  (void)width;
  const int s = hipcpu::lane() - d;
  return hipcpu::exchange(x, s < 0 ? hipcpu::lane() : s);
}
inline unsigned long long __ballot(int pred) {
  hipcpu::WaveCtx& w = hipcpu::wave();
  w.buf[hipcpu::lane()] = pred ? 1u : 0u;
  w.bar->arrive_and_wait();
  unsigned long long m = 0;
  for (int i = 0; i < 64; i++)
    if (w.buf[i]) m |= 1ull << i;
  w.bar->arrive_and_wait();
  return m;
}

// ---- lane moves (gfx950 semantics, checked on the GPU for the controls used)
// DPP move: quad_perm (0x00-0xFF), row_shl:s (0x101-0x10F), row_shr:s
// (0x111-0x11F), row_ror:s (0x121-0x12F), row_mirror (0x140); rows are 16
// lanes; a source outside the row leaves `old` (bound_ctrl off, full masks).
// DPP lane moves as the gfx9 ISA defines them: a lane whose source lies out
// of its row (or of the wave), or whose row is off in row_mask, keeps `old`
// (bound_ctrl off).  row_bcast:15 takes lane 15 of the previous row,
// row_bcast:31 lane 31.
inline uint32_t __builtin_amdgcn_update_dpp(uint32_t old, uint32_t src, int ctrl, int row_mask, int bank_mask, bool) {
  const int l = hipcpu::lane(), row = l & ~15, r = l & 15;
  int s = -1;
  if (ctrl <= 0xFF) s = (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);
  else if (ctrl >= 0x101 && ctrl <= 0x10F) s = r + (ctrl - 0x100) < 16 ? l + (ctrl - 0x100) : -1;
  else if (ctrl >= 0x111 && ctrl <= 0x11F) s = r - (ctrl - 0x110) >= 0 ? l - (ctrl - 0x110) : -1;
  else if (ctrl >= 0x121 && ctrl <= 0x12F) s = row | ((r + (ctrl - 0x120)) & 15);
  else if (ctrl == 0x140) s = row | (15 - r);
  else if (ctrl == 0x142) s = row >= 16 ? row - 1 : -1;
  else if (ctrl == 0x143) s = 31;
  else std::abort();
  if (!((row_mask >> (l >> 4)) & 1) || !((bank_mask >> (r >> 2)) & 1)) s = -1;
  const uint32_t v = hipcpu::exchange(src, s < 0 ? l : s);
  return s < 0 ? old : v;
}
struct hipcpu_u2 {
  uint32_t v[2];
  uint32_t operator[](int i) const { return v[i]; }
};
// v_permlane16_swap: odd rows of the first operand swap with even rows of
// the second; v_permlane32_swap: the upper half of the first with the lower
// half of the second.  Returns {first, second} after the swap.
inline hipcpu_u2 __builtin_amdgcn_permlane16_swap(uint32_t a, uint32_t b, bool, bool) {
  const int l = hipcpu::lane();
  const uint32_t a_up = hipcpu::exchange(a, l < 48 ? l + 16 : l);  // a of lane + 16
  const uint32_t b_dn = hipcpu::exchange(b, l >= 16 ? l - 16 : l);  // b of lane - 16
  const bool odd = (l >> 4) & 1;
  return {{odd ? b_dn : a, odd ? b : a_up}};
}
inline hipcpu_u2 __builtin_amdgcn_permlane32_swap(uint32_t a, uint32_t b, bool, bool) {
  const int l = hipcpu::lane();
  const uint32_t a_up = hipcpu::exchange(a, l < 32 ? l + 32 : l);
  const uint32_t b_dn = hipcpu::exchange(b, l >= 32 ? l - 32 : l);
  const bool hi = l >= 32;
  return {{hi ? b_dn : a, hi ? b : a_up}};
}
inline uint32_t __builtin_amdgcn_mbcnt_lo(uint32_t mask, uint32_t acc) {
  const int l = hipcpu::lane();
  return acc + (uint32_t)__builtin_popcount(l >= 32 ? mask : (mask & ((1u << l) - 1u)));
}
inline uint32_t __builtin_amdgcn_mbcnt_hi(uint32_t mask, uint32_t acc) {
  const int l = hipcpu::lane();
  return acc + (uint32_t)(l < 32 ? 0 : __builtin_popcount(mask & ((1u << (l - 32)) - 1u)));
}
template <typename T>
inline T __builtin_amdgcn_readlane(T x, int l) { return hipcpu::exchange(x, l); }
// The kernels call it with every lane of the wave active: lane 0 is the first.
template <typename T>
inline T __builtin_amdgcn_readfirstlane(T x) { return hipcpu::exchange(x, 0); }
// A wave-wide barrier stands in for the code-motion barrier; the fences order
// nothing further on the host.
inline void __builtin_amdgcn_wave_barrier() { hipcpu::wave().bar->arrive_and_wait(); }
#define __builtin_amdgcn_fence(...) ((void)0)

inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }

inline int __popc(unsigned x) { return __builtin_popcount(x); }
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
inline int __ffsll(long long x) { return __builtin_ffsll(x); }
inline int __clzll(long long x) { return x ? __builtin_clzll((unsigned long long)x) : 64; }
inline unsigned long long __umul64hi(unsigned long long a, unsigned long long b) {
  return (unsigned long long)(((unsigned __int128)a * b) >> 64);
}
inline float __uint_as_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

template <typename T, typename U>
inline T atomicAdd(T* p, U v) { return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST); }
inline int atomicCAS(int* p, int cmp, int val) {
  __atomic_compare_exchange_n(p, &cmp, val, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
  return cmp;
}
inline unsigned atomicOr(unsigned* p, unsigned v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }
inline int atomicMin(int* p, int v) {
  int cur = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while (v < cur && !__atomic_compare_exchange_n(p, &cur, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {
  }
  return cur;
}

// Scoped atomics: device memory is host memory, so every scope is the
// process; s_waitcnt has nothing to wait for.
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
template <typename T>
inline void __hip_atomic_store(T* p, T v, int, int) { __atomic_store_n(p, v, __ATOMIC_SEQ_CST); }
template <typename T>
inline T __hip_atomic_load(const T* p, int, int) { return __atomic_load_n(p, __ATOMIC_SEQ_CST); }
template <typename T, typename U>
inline T __hip_atomic_fetch_add(T* p, U v, int, int) { return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST); }
inline void __builtin_amdgcn_s_waitcnt(int) {}
inline void __builtin_amdgcn_s_sleep(int) { std::this_thread::yield(); }

// ---- runtime API on host memory ----
inline int& hipcpu_last_error() {
  static int e = 0;
  return e;
}
inline hipError_t hipGetLastError() { int e = hipcpu_last_error(); hipcpu_last_error() = 0; return e; }
inline const char* hipGetErrorString(hipError_t e) { return e ? "hipcpu error" : "no error"; }
template <typename T>
inline hipError_t hipMalloc(T** p, size_t n) {
  *p = (T*)std::malloc(n ? n : 1);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipFree(void* p) { std::free(p); return hipSuccess; }
inline hipError_t hipMemset(void* p, int v, size_t n) { std::memset(p, v, n); return hipSuccess; }
inline hipError_t hipMemcpy(void* d, const void* s, size_t n, int) { std::memcpy(d, s, n); return hipSuccess; }
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
typedef int hipStreamCaptureStatus;
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* s) {
  *s = hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipGetDeviceCount(int* n) { *n = 1; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, int attr, int) {
  *v = attr == hipDeviceAttributeMultiprocessorCount ? 256 : 163840;
  return hipSuccess;
}
inline hipError_t hipFuncSetAttribute(const void*, int, int) { return hipSuccess; }
template <class F>
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, F, int, size_t) { *n = 8; return hipSuccess; }
// A __device__ variable is a host variable here: its symbol is its address.
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
  *p = const_cast<void*>(sym);
  return hipSuccess;
}
