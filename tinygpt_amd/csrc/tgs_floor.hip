// tgs_floor.hip -- the plain-read floor of the fused top_k <= 64 kernel, for
// measurement only (bench.py --workload read; built into its own library,
// libtgs_floor.so, not into the sampler's C ABI).
//
// It reads [B] rows of V fp32 logits with the fused kernel's grid and load
// pattern: S chunks per row of L ids, one workgroup of K64_NT threads per
// chunk, thread t issuing its K64_NVT non-temporal 16-byte loads (chunk
// vectors t, t + K64_NT, ...) at entry, and keeps only what the loads need to
// stay live: the maximum of each chunk, written out.  The time of a launch is
// the floor the sampling chain adds its work to.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tgs_kernels.h"

namespace {

constexpr int NT = tgs::K64_NT;
constexpr int NVT = tgs::K64_NVT;

__global__ __launch_bounds__(NT) void floor_read_kernel(const float* x, int V, long long stride, int S, int L,
                                                        float* out) {
  const int b = (int)blockIdx.x / S, c = (int)blockIdx.x % S;
  const int v0 = c * L, v1 = min(V, v0 + L);
  const int nvec = (v1 - v0) / 4;
  const float* rowp = x + (long long)b * stride + v0;
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  v4u raw[NVT];
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    const int j = (int)threadIdx.x + i * NT;
    raw[i] = __builtin_nontemporal_load((const v4u*)(rowp + 4 * (j < nvec ? j : nvec - 1)));
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    m = fmaxf(m, fmaxf(fmaxf(__uint_as_float(raw[i].x), __uint_as_float(raw[i].y)),
                       fmaxf(__uint_as_float(raw[i].z), __uint_as_float(raw[i].w))));
  }
  for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  __shared__ float wm[NT / 64];
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = wm[0];
    for (int i = 1; i < NT / 64; i++) r = fmaxf(r, wm[i]);
    out[blockIdx.x] = r;
  }
}

}  // namespace

extern "C" {

// Reads rows [B][V] (stride `stride` floats) of a 16-byte aligned fp32 array
// in S chunks per row; out: [B * S] chunk maxima.  Returns 0, or -1 when the
// shape does not fit the pattern (V and stride multiples of 4, a chunk of at
// most K64_NT * K64_NVT vectors), -2 on a launch error.
int tgs_floor_read(const float* x, int B, int V, long long stride, int S, float* out, void* stream) {
  if (!x || !out || B < 1 || V < 4 || V % 4 != 0 || stride < V || stride % 4 != 0 || S < 1) return -1;
  if ((uintptr_t)x % 16 != 0) return -1;
  const int L = ((V + S - 1) / S + 3) / 4 * 4;
  if ((V + L - 1) / L != S || L / 4 > NT * NVT) return -1;
  hipLaunchKernelGGL(floor_read_kernel, dim3(B * S), dim3(NT), 0, (hipStream_t)stream, x, V, stride, S, L, out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
