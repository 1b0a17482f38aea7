// numerics.cpp -- checks, on the CPU, that the device arithmetic shortcuts of
// tgs_device.h equal the canonical operations they replace, over the input
// ranges the kernels feed them.  The header is compiled unchanged (host
// shim).  TEST INFRASTRUCTURE ONLY.
//   numerics div N seed   tg_div_rcp(a, b, 1/b) == a / b, a in [0, 1], b in [1, 2^18]
//   numerics exp N seed   tg_expf_nonpos(x) == tg_expf(x), x <= 0, -inf, NaN
//   numerics q40 N seed   (u64)tg_q40d(e) == tg_q40(e), e in [0, 1]
//   numerics divt N seed  tg_div_t(z, T, 1/T) == z / T, any z, T > 0 with 1/T finite
//   numerics q40exp N seed  tg_q40d_exp_nonpos(x) == tg_q40d(tg_expf_nonpos(x))
//   numerics pow2fma N seed the mass and the weight of fma(z, rT, -m) == those of
//                           RN(z rT) - m, T a power of two, m = RN(zmax rT), zmax >= z
// Prints the number of mismatches (and the first few).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <random>
#include <string>

#include "tgs_device.h"

using namespace tgs;

static float bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
static uint32_t ubits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char** argv) {
  if (argc < 4) return 2;
  const std::string mode = argv[1];
  const long long N = std::atoll(argv[2]);
  std::mt19937_64 g(std::strtoull(argv[3], nullptr, 10));
  long long bad = 0;
  auto report = [&](const char* what, float x, float y, double r0, double r1) {
    if (++bad <= 5) std::printf("mismatch %s %a %a: %a vs %a\n", what, x, y, r0, r1);
  };
  if (mode == "div") {
    // weights a: every exponent from 2^-48 to 1 (and 0, 1); denominators b in [1, 2^18]
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      float a, b;
      const int ea = (int)(r % 49), eb = (int)((r >> 8) % 19);
      const uint32_t ma = (uint32_t)(r >> 16) & 0x7FFFFFu, mb = (uint32_t)(r >> 40) & 0x7FFFFFu;
      a = bits(((uint32_t)(127 - ea) << 23) | ma);
      if (a > 1.0f) a = 1.0f;
      b = bits(((uint32_t)(127 + eb) << 23) | mb);
      switch (i & 15) {
        case 0: a = 0.0f; break;
        case 1: a = 1.0f; break;
        case 2: b = bits(((uint32_t)(127 + eb) << 23) | 0x7FFFFFu); break;
        case 3: a = bits(((uint32_t)(127 - ea) << 23) | 0x7FFFFFu); if (a > 1.0f) a = 1.0f; break;
        case 4: b = bits((uint32_t)(127 + eb) << 23); break;
        case 5: a = tg_expf(-(float)(r % 32000) * 0.001f); break;
        default: break;
      }
      const float rb = 1.0f / b;
      const float q1 = tg_div_rcp(a, b, rb), q0 = a / b;
      if (ubits(q1) != ubits(q0)) report("div", a, b, q1, q0);
    }
  } else if (mode == "exp") {
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      float x;
      if ((i & 3) == 0) x = -bits((uint32_t)r & 0x7FFFFFFFu);               // any non-positive bit pattern
      else x = -(float)((double)(r >> 11) * 0x1p-53 * 40.0);                 // uniform in [-40, 0]
      if (i == 0) x = -__builtin_inff();
      if (i == 1) x = bits(0x7FC00000u);
      if (i == 2) x = -0.0f;
      if (i == 3) x = 0.0f;
      if (i == 4) x = -32.0f;
      const float e1 = tg_expf_nonpos(x), e0 = tg_expf(x);
      if (ubits(e1) != ubits(e0)) report("exp", x, 0, e1, e0);
    }
  } else if (mode == "q40") {
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      float e = (i & 1) ? tg_expf(-(float)((double)(r >> 11) * 0x1p-53 * 33.0))
                        : bits(((uint32_t)(127 - (int)(r % 60)) << 23) | ((uint32_t)(r >> 20) & 0x7FFFFFu));
      if (e > 1.0f) e = 1.0f;
      if (i == 0) e = 0.0f;
      if (i == 1) e = 1.0f;
      const u64 q1 = (u64)tg_q40d(e), q0 = tg_q40(e);
      if (q1 != q0) report("q40", e, 0, (double)q1, (double)q0);
    }
  } else if (mode == "q40exp") {
    // x <= 0 (every non-positive bit pattern, uniform [-40, 0], the region
    // around the -32 and -27.73 cut-offs, specials) and tiny positive x.
    // NaNs are quiet: the kernels pass the result of a subtraction or a
    // fused multiply-add, never a signalling NaN (for which the host's
    // fmaxf returns NaN).
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      float x;
      switch (i & 3) {
        case 0: {
          uint32_t u = (uint32_t)r & 0x7FFFFFFFu;
          if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) u |= 0x400000u;
          x = -bits(u);
          break;
        }
        case 1: x = -(float)((double)(r >> 11) * 0x1p-53 * 40.0); break;
        case 2: x = -27.0f - (float)((double)(r >> 11) * 0x1p-53 * 6.0); break;
        default: x = -(float)((double)(r >> 11) * 0x1p-53 * 2.0); break;
      }
      if (i == 0) x = -__builtin_inff();
      if (i == 1) x = bits(0x7FC00000u);
      if (i == 2) x = -0.0f;
      if (i == 3) x = 0.0f;
      if (i == 4) x = -32.0f;
      if (i == 5) x = bits(1u);
      if (i == 6) x = bits(0x00800000u);
      const double q1 = tg_q40d_exp_nonpos(x), q0 = tg_q40d(tg_expf_nonpos(x));
      if (q1 != q0) report("q40exp", x, 0, q1, q0);
    }
  } else if (mode == "pow2fma") {
    // a power-of-two temperature: the mass of y - m with y = z rT and the
    // maximum m = RN(zmax rT), zmax >= z, equals the mass of the fused
    // fma(z, rT, -m) (z rT is exact there except below the normal range,
    // where both differences round to the same weight)
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      const int et = (int)((r >> 8) % 41) - 20;
      const float T = bits((uint32_t)(127 + et) << 23);
      const float rT = 1.0f / T;
      const int ez = (int)(r % 300) - 150;
      const uint32_t mz = (uint32_t)(r >> 16) & 0x7FFFFFu;
      float z = (ez <= -127) ? bits(mz >> (uint32_t)(-126 - ez > 23 ? 23 : -126 - ez))
                             : bits(((uint32_t)(127 + (ez > 127 ? 127 : ez)) << 23) | mz);
      if ((r >> 62) & 1) z = -z;
      float dz = bits(((uint32_t)(127 + (int)((r >> 40) % 40) - 30) << 23) | ((uint32_t)(r >> 20) & 0x7FFFFFu));
      switch ((r >> 56) & 7) {
        case 0: dz = 0.0f; break;
        case 1: dz = bits((uint32_t)(r >> 30) & 0xFFu); break;  // a few denormal ulps
        case 2: z = -__builtin_inff(); break;
        case 3: z = bits(0x7FC00000u); break;
        default: break;
      }
      const float zmax = (z == z && z > -__builtin_inff()) ? z + dz : 1.0f;
      if (!(zmax >= z) && z == z && z > -__builtin_inff()) continue;
      const float m = zmax * rT;
      if (!__builtin_isfinite(m)) continue;
      const float x1 = __builtin_fmaf(z, rT, -m), x0 = z * rT - m;
      const double q1 = tg_q40d_exp_nonpos(x1);
      const double q0 = tg_q40d(tg_expf_nonpos(x0));
      if (q1 != q0) report("pow2fma", z, T, q1, q0);
      // the weight itself (the residual draw's operand), bit for bit
      const float e1 = tg_expf_nonpos(x1), e0 = tg_expf_nonpos(x0);
      if (ubits(e1) != ubits(e0)) report("pow2fma-w", z, T, e1, e0);
    }
  } else if (mode == "divt") {
    // z: every exponent of the fast range and beyond it, both signs, plus
    // specials; T: every exponent from 2^-24 to 2^24 (around the fast range),
    // including the powers of two and all-ones mantissas
    for (long long i = 0; i < N; i++) {
      const uint64_t r = g();
      const int ez = (int)(r % 80) - 40, et = (int)((r >> 8) % 49) - 24;
      const uint32_t mz = (uint32_t)(r >> 16) & 0x7FFFFFu, mt = (uint32_t)(r >> 40) & 0x7FFFFFu;
      float z = bits(((uint32_t)(127 + ez) << 23) | mz);
      if ((r >> 63) & 1) z = -z;
      float T = bits(((uint32_t)(127 + et) << 23) | mt);
      switch (i & 31) {
        case 0: z = 0.0f; break;
        case 1: z = -0.0f; break;
        case 2: z = __builtin_inff(); break;
        case 3: z = -__builtin_inff(); break;
        case 4: z = bits(0x7FC00000u); break;
        case 5: z = bits((uint32_t)(r >> 20) & 0x7FFFFFu); break;  // denormal
        case 6: T = bits((uint32_t)(127 + et) << 23); break;        // power of two
        case 7: T = bits(((uint32_t)(127 + et) << 23) | 0x7FFFFFu); break;
        case 8: z = bits(((uint32_t)(127 + ez) << 23) | 0x7FFFFFu); break;
        case 9: z = (float)((int)(r % 2001) - 1000) * 0.01f; T = (float)(1 + (r >> 32) % 200) * 0.01f; break;
        case 10: T = bits(((uint32_t)(127 - 126) << 23) | mt); break;  // T near the smallest normal
        case 11: z = bits(((uint32_t)(127 + 100) << 23) | mz); break;  // large logits
        default: break;
      }
      const float rT = 1.0f / T;
      if (!__builtin_isfinite(rT)) continue;
      const float q1 = tg_div_t(z, T, rT, tg_div_t_mode(T)), q0 = z / T;
      if (ubits(q1) != ubits(q0) && !(q0 != q0 && q1 != q1)) report("divt", z, T, q1, q0);
    }
  } else {
    return 2;
  }
  std::printf("%s %lld checked, %lld mismatches\n", mode.c_str(), N, bad);
  return bad ? 1 : 0;
}
