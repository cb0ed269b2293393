// synth.hip -- the measurement protocol's synthetic inputs on the GPU.
//
// A counter-based generator: element i of stream `seed` is a pure function
// of (seed, i), so a tensor is the same whatever grid makes it, and the CPU
// oracle (oracle/oracle.c, loom_oracle_synth) makes the same bits with the
// same operations in the same order.  splitmix64's finaliser mixes
// seed * K1 + i * K2; uniform: the top 24 bits * 2^-24 (exact), scaled to
// [a, b); normal: Box-Muller, n = sqrt(-2 ln u1) cos(2 pi u2) with u1 in
// (0, 1] and u2 in [0, 1) from two 24-bit fields, scaled to N(a, b).  ln and
// cos are polynomials written here (not the device math library, whose
// last-place rounding differs from the host's): ln from the exponent and the
// odd series of ln((1+s)/(1-s)) on a mantissa in [sqrt(1/2), sqrt(2)); cos
// (2 pi u2) from an exact octant split of u2 and Taylor polynomials of sin
// and cos on [0, pi/4].  Every multiply-add is an explicit fmaf, no other
// contraction is allowed, division is the correctly rounded form and the
// square root is computed in integer arithmetic, so every step rounds exactly
// as the host's.  bf16 output: round to nearest even.  No counterpart in the
// reference.
#include "common.h"

#pragma clang fp contract(off)

namespace {

LOOM_DEV uint64_t synth_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

LOOM_DEV float synth_ln(float x) {   // x in [2^-24, 1]
  uint32_t b = __float_as_uint(x);
  int e = (int)((b >> 23) & 0xff) - 127;
  float m = __uint_as_float((b & 0x007fffffu) | 0x3f800000u);   // [1, 2)
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = __fdiv_rn(m - 1.0f, m + 1.0f);
  const float s2 = s * s;
  float p = fmaf(s2, 0.11111111f, 0.14285715f);
  p = fmaf(s2, p, 0.2f);
  p = fmaf(s2, p, 0.33333334f);
  p = fmaf(s2, p, 1.0f);
  const float lnm = 2.0f * s * p;
  return fmaf((float)e, 0.69314718f, lnm);
}

LOOM_DEV float synth_sin(float a) {   // a in [0, pi/4]
  const float a2 = a * a;
  float p = fmaf(a2, -2.5052108e-8f, 2.7557319e-6f);
  p = fmaf(a2, p, -1.9841270e-4f);
  p = fmaf(a2, p, 8.3333333e-3f);
  p = fmaf(a2, p, -1.6666667e-1f);
  return fmaf(a * a2, p, a);
}
LOOM_DEV float synth_cos(float a) {
  const float a2 = a * a;
  float p = fmaf(a2, 2.0876757e-9f, -2.7557319e-7f);
  p = fmaf(a2, p, 2.4801587e-5f);
  p = fmaf(a2, p, -1.3888889e-3f);
  p = fmaf(a2, p, 4.1666667e-2f);
  p = fmaf(a2, p, -0.5f);
  return fmaf(a2, p, 1.0f);
}

LOOM_DEV float synth_cos2pi(float t) {   // t = k 2^-24
  const float t8 = t * 8.0f;
  const int o = (int)t8;
  const float f = t8 - (float)o;
  const int k = o >> 1;
  if ((o & 1) == 0) {
    const float a = f * 0.78539816f;
    return k == 0 ? synth_cos(a) : k == 1 ? -synth_sin(a) : k == 2 ? -synth_cos(a) : synth_sin(a);
  }
  const float a = (1.0f - f) * 0.78539816f;
  return k == 0 ? synth_sin(a) : k == 1 ? -synth_cos(a) : k == 2 ? -synth_sin(a) : synth_cos(a);
}

// sqrt(x) rounded to nearest, for x = 0 or a positive normal float, in
// integer arithmetic: v_sqrt_f32 is not correctly rounded, and the host must
// get the same bits.  x = M 2^E with M in [2^24, 2^26) and E even,
// R = floor(sqrt(M 2^24)) has 25 bits (a floating-point estimate corrected by
// integer steps, so the estimate's accuracy does not matter), and the 24-bit
// significand is R / 2 rounded by R's last bit (a square root of a float is
// never halfway between two floats).
LOOM_DEV float synth_sqrt(float x) {
  if (!(x > 0.0f)) return 0.0f;
  const uint32_t bx = __float_as_uint(x);
  uint64_t m = (bx & 0x007fffffu) | 0x00800000u;
  int e = (int)((bx >> 23) & 0xff) - 150;
  if (e & 1) {
    m <<= 1;
    e -= 1;
  } else {
    m <<= 2;
    e -= 2;
  }
  const uint64_t n = m << 24;
  uint64_t r = (uint64_t)sqrt((double)n);
  while (r * r > n) --r;
  while ((r + 1) * (r + 1) <= n) ++r;
  const uint64_t q = (r >> 1) + (r & 1);
  return ldexpf((float)q, (e - 24) / 2 + 1);
}

template <bool BF16>
__global__ void __launch_bounds__(256) synth_kernel(void* out, int64_t n, uint64_t seed, int dist,
                                                    float a, float b) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t z = synth_mix(seed * 0xD1B54A32D192ED03ull + (uint64_t)i * 0x9E3779B97F4A7C15ull);
    float v;
    if (dist == 0) {
      v = fmaf(b - a, (float)(z >> 40) * 0x1p-24f, a);
    } else {
      const float u1 = (float)((z >> 40) + 1) * 0x1p-24f;
      const float u2 = (float)((z >> 16) & 0xffffffu) * 0x1p-24f;
      const float r = synth_sqrt(-2.0f * synth_ln(u1));
      v = fmaf(b, r * synth_cos2pi(u2), a);
    }
    if constexpr (BF16)
      static_cast<uint16_t*>(out)[i] = (uint16_t)f2bf(v);
    else
      static_cast<float*>(out)[i] = v;
  }
}

}  // namespace

extern "C" {

int loom_hip_synth(void* out, int64_t n, uint64_t seed, int dist, float a, float b, int bf16,
                   void* stream, char* err, size_t errlen) {
  if (!out || n < 0 || (dist != 0 && dist != 1))
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "synth: a non-null output, n >= 0 and dist 0 (uniform) or 1 (normal)");
  if (n == 0) return loom_ok(err, errlen);
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (bf16)
    hipLaunchKernelGGL(synth_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, out, n, seed,
                       dist, a, b);
  else
    hipLaunchKernelGGL(synth_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, out, n, seed,
                       dist, a, b);
  return loom_check_launch(err, errlen, "synth");
}

}  // extern "C"
