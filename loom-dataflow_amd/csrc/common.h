// common.h -- shared device helpers and host-side error plumbing for the
// loom_hip kernels (gfx950 only).
//
// bf16 tensors travel as raw 16-bit patterns (uint16_t); conversion to fp32
// is exact (bits << 16) and conversion back is round-to-nearest-even with
// NaNs quieted, the same rounding the CPU oracle applies, so a value the
// kernel and the oracle compute identically in fp32 stores identically.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>

// ---------------------------------------------------------------------------
// vector types for the gfx950 bf16 MFMA builtins
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define LOOM_DEV __device__ __forceinline__

LOOM_DEV float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
LOOM_DEV float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }
LOOM_DEV float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

LOOM_DEV uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// two fp32 -> one dword holding (lo = bf16(a), hi = bf16(b))
LOOM_DEV uint32_t pack_bf16x2(float a, float b) { return f2bf(a) | (f2bf(b) << 16); }

// D[16x16] += A[16x32] . B[32x16]; lane l supplies row (A) / column (B)
// l % 16 and eight consecutive k of group l / 16; D lands as rows
// 4*(l/16) + i, column l % 16.
LOOM_DEV f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Pack the low (pack_lo) or high (pack_hi) 16-bit halves of two dwords:
// result low half from x, high half from y.
LOOM_DEV uint32_t pack_lo(uint32_t x, uint32_t y) { return (x & 0xffffu) | (y << 16); }
LOOM_DEV uint32_t pack_hi(uint32_t x, uint32_t y) { return (x >> 16) | (y & 0xffff0000u); }

// 8x8 transpose of 16-bit elements held as 8 rows of u32x4 (row r = eight
// consecutive columns).  Output column c = eight consecutive rows.
LOOM_DEV void transpose8x8(const u32x4_t (&in)[8], u32x4_t (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {      // dword j of each row holds columns 2j, 2j+1
#pragma unroll
    for (int i = 0; i < 4; ++i) {    // rows 2i, 2i+1
      out[2 * j][i] = pack_lo(in[2 * i][j], in[2 * i + 1][j]);
      out[2 * j + 1][i] = pack_hi(in[2 * i][j], in[2 * i + 1][j]);
    }
  }
}

LOOM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Map a linear workgroup id so that each of the 8 XCDs (which receive ids
// round-robin) owns one contiguous range of the logical id space: logical
// neighbours then share an L2.
LOOM_DEV int xcd_remap(int bid, int nblocks) {
  const int nx = 8;
  if (nblocks % nx != 0) return bid;
  return (bid % nx) * (nblocks / nx) + bid / nx;
}

// ---------------------------------------------------------------------------
// host-side error reporting through the C ABI's (err, errlen) pair
// ---------------------------------------------------------------------------
enum {
  LOOM_OK = 0,
  LOOM_EINVAL = 1,    // shapes, tiles, pointers or workspace rejected
  LOOM_EUNSUP = 2,    // legal in the reference but not built for gfx950 here
  LOOM_EHIP = 3,      // HIP runtime reported an error
};

static inline int loom_fail(char* err, size_t errlen, int code, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return code;
}

static inline int loom_ok(char* err, size_t errlen) {
  if (err && errlen) err[0] = '\0';
  return LOOM_OK;
}

static inline int loom_check_launch(char* err, size_t errlen, const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return loom_fail(err, errlen, LOOM_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return loom_ok(err, errlen);
}

static inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
