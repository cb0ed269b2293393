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
#include <atomic>
#include <initializer_list>

#include "../../include/loom_hip.h"   // every entry point matches its declaration

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

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// two fp32 -> one dword holding (lo = bf16(a), hi = bf16(b)): gfx950's
// v_cvt_pk_bf16_f32, round to nearest even (the same bits as f2bf for every
// non-NaN input)
LOOM_DEV uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// D[16x16] += A[16x32] . B[32x16]; lane l supplies row (A) / column (B)
// l % 16 and eight consecutive k of group l / 16; D lands as rows
// 4*(l/16) + i, column l % 16.
LOOM_DEV f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// 16-bit element type: kernels are templated on H (false = bf16, true =
// IEEE f16, the reference's own element type).  Both travel as raw 16-bit
// patterns; only the MFMA, the fp32 -> 16-bit rounding (round to nearest
// even in both cases) and the 16-bit -> fp32 widening differ.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <bool H>
LOOM_DEV f32x4_t mfma16t(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (H)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return mfma16(a, b, c);
}
// two fp32 -> one dword (lo = a, hi = b) in the element type
template <bool H>
LOOM_DEV uint32_t pack2(float a, float b) {
  if constexpr (H)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
  else
    return pack_bf16x2(a, b);
}
// one fp32 -> element bits
template <bool H>
LOOM_DEV uint32_t cvt16(float a) {
  if constexpr (H)
    return __builtin_bit_cast(uint16_t, (_Float16)a);
  else
    return f2bf(a);
}
// low / high element of a dword -> fp32 (exact)
template <bool H>
LOOM_DEV float lo16(uint32_t w) {
  if constexpr (H)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  else
    return bf2f_lo(w);
}
template <bool H>
LOOM_DEV float hi16(uint32_t w) {
  if constexpr (H)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  else
    return bf2f_hi(w);
}
// a dword holding two 1.0s
template <bool H>
constexpr uint32_t kOnePair = H ? 0x3C003C00u : 0x3F803F80u;

// Pack the low (pack_lo) or high (pack_hi) 16-bit halves of two dwords:
// result low half from x, high half from y.  One v_perm_b32 each: the
// selector picks bytes of the 64-bit value {y, x} (x = bytes 0-3).
LOOM_DEV uint32_t pack_lo(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
LOOM_DEV uint32_t pack_hi(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

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

// Set (per thread) by loom_hip_check_variant: entry points validate their
// arguments and return before launching anything.
bool& loom_validate_only_flag();
static inline bool loom_validate_only() { return loom_validate_only_flag(); }

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

// CU count of the device `st` belongs to (the null stream: the current
// device), cached per device; 0 when unknown.
inline int stream_cus(hipStream_t st) {
  static std::atomic<int> cache[64];   // count + 1; 0 = not queried yet
  int dev = 0;
  if (st != nullptr) {
    hipDevice_t d = 0;
    if (hipStreamGetDevice(st, &d) != hipSuccess) return 0;
    dev = (int)d;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return 0;
  }
  if (dev < 0 || dev >= 64) return 0;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    c = n + 1;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c - 1;
}

// Whether the product of non-negative extents stays within `limit`, computed
// without signed overflow (caller-supplied extents can be anything).
static inline bool loom_prod_le(std::initializer_list<int64_t> xs, int64_t limit) {
  int64_t p = 1;
  for (int64_t x : xs) {
    if (x < 0 || __builtin_mul_overflow(p, x, &p) || p > limit) return false;
  }
  return true;
}
static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The reference bounds every loom.sym by the extent of the loop it tiles
// (its upper_bound, exported as natural_ub:
// lib/passes/lcs/src/staged_etg_builder.cpp:1420-1430) and aligns the inner
// dimensions of its tiles to 32 (lib/passes/lcs/src/hw_alignment.cpp:16).
// The gfx950 analogue of that alignment is the 16-element MFMA edge: a tiled
// symbol takes any multiple of 16 up to its extent, or the extent itself.
// The kernels' results do not depend on the workgroup tile (every output
// element accumulates in the same order whatever tile holds it), so a bound
// value runs on the nearest built tile.  Returns, given the tiles built for
// the axis (`built`, ascending):
//   > 0  the smallest built tile >= t, or the largest built tile when t is
//        larger than every built one;
//     0  t exceeds the extent (callers return LOOM_EINVAL);
//    -1  t is neither a multiple of 16 nor the whole extent (LOOM_EINVAL).
constexpr int64_t kLoomTileAlign = 16;
static inline int64_t loom_fit_tile(int64_t t, int64_t extent, const int64_t* built, int nbuilt) {
  if (t > extent) return 0;
  if (t % kLoomTileAlign != 0 && t != extent) return -1;
  for (int i = 0; i < nbuilt; ++i)
    if (built[i] >= t) return built[i];
  return built[nbuilt - 1];
}

// ---------------------------------------------------------------------------
// raw buffer loads: range-checked by the hardware against `bytes` (reads past
// the end return zeros and issue no memory request), so guarded loads need
// no branch
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// The descriptor must be wave-uniform; readfirstlane states that to the
// compiler, which otherwise may keep it in VGPRs and wrap every buffer
// instruction in a waterfall loop.
LOOM_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}
LOOM_DEV u32x4_t buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
LOOM_DEV u32x2_t buf_load8(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
LOOM_DEV uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
LOOM_DEV uint32_t buf_load2(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Elements key .. key+7 of row d of a [rows][n] tensor of 16-bit values
// whose rows need not start on 16-byte boundaries (n not a multiple of 8),
// through the buffer descriptor r over the whole tensor (n * rows * 2 <
// 2^31).  A piece inside its row is one 16-byte load at whatever 2-byte
// aligned offset it starts: ROCm's driver runs every GPU process in the
// unaligned access mode (SH_MEM_CONFIG.alignment_mode UNALIGNED), where
// dword and wider loads take any byte address.  A load reaching past the
// buffer's range returns zeros whole, so a piece that reaches past its row's
// end (past the tensor for the last row) takes one 2-byte load per element
// (the elements past the row are the next row's, past the tensor zeros); a
// piece wholly past the row is zero.
LOOM_DEV u32x4_t row_piece8(rsrc_t r, int n, int d, int key) {
  const uint32_t off = (uint32_t)(d * n + key) * 2;
  if (key + 8 <= n) return buf_load16(r, off);
  if (key >= n) return u32x4_t{0u, 0u, 0u, 0u};
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = buf_load2(r, off + 2 * e);
  return u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                 h[6] | (h[7] << 16)};
}

LOOM_DEV float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
LOOM_DEV float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// ---------------------------------------------------------------------------
// gfx950 LDS DMA and transpose reads
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) char lds_char_t;
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's data lands at lds + 16 l, where lds
// must be the same for the whole wave.  No range check: callers clamp.
// Issued from inline assembly so the compiler does not track it: its LDS-DMA
// tracking holds only a few loads in flight and beyond that waits for all of
// them before any LDS read.  Callers therefore order it themselves with
// LOOM_WAIT_VMCNT + barrier_nofence before reading the destination.  M0 holds
// the LDS address; one wait state separates the M0 write from its use.
LOOM_DEV uint32_t lds_addr(const lds_char_t* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
LOOM_DEV void dma_load16(const void* g, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(g), "s"(lds)
      : "memory", "m0");
}

// 1 KB of zeros in device memory: the source of the LDS-DMA copies of
// padding rows (an operand narrower than the tile built for it), so those
// rows hold zeros and every wave still issues the same copies per stage.
static __device__ __align__(1024) uint32_t loom_zero_kb[256] = {};

// LDS banks repeat every 256 bytes.  A transposed read (below) serves 32
// lanes per pass; when each of its 16-lane groups reads rows r..r+3 of one
// tile and the two groups rows r+4..r+7, the pass touches 32-byte pieces of 8
// consecutive rows, and rows that sit at the same offset of the 256-byte
// window must take distinct 16-byte chunk pairs.  tr_swz(k, rb) is the XOR a
// row k of rb bytes (a multiple of 32) applies to its chunk index.  With
// g = gcd(rb, 256), rows 256/g apart share a window offset and g/32 of them
// fall among 8 consecutive rows; the XOR takes g/32 values below g/16, and
// since rb is a multiple of g it keeps every chunk index inside its row.
// g and pr are powers of two, so the division and the modulo are a shift and
// a mask (k >= 0): no integer-division sequence when rb is only known at run
// time.
LOOM_DEV int tr_swz(int k, int rb) {
  const int g = (rb & -rb) < 256 ? (rb & -rb) : 256;  // gcd(rb, 256)
  const int pr = g >= 32 ? g / 32 : 1;                 // rows of a pass sharing an offset
  return 2 * ((k >> (8 - __builtin_ctz(g))) & (pr - 1));   // (k / (256 / g)) % pr
}

// ds_read_b64_tr_b16: in each 16-lane group, lanes 4a..4a+3 address the four
// 8-byte pieces of row a of a 4x16 matrix of 16-bit values; lane j receives
// column j, (row0[j], row1[j], row2[j], row3[j]).
LOOM_DEV u32x2_t lds_read_tr16(const lds_char_t* p) {
  return __builtin_bit_cast(
      u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                   (__attribute__((address_space(3))) s16x4_t*)(p)));
}

// ---------------------------------------------------------------------------
// MFMAs with the accumulator pinned to AGPRs.  Written as inline assembly
// because, with 64 accumulator chains live across an unrolled loop, the
// register allocator otherwise splits some of them into VGPRs and copies
// them back and forth around every MFMA.  The compiler's hazard recognizer
// does not see these instructions: callers let the MFMAs retire (s_nop)
// before reading an accumulator with any other instruction, and after
// writing one before the first MFMA that reads it.
// ---------------------------------------------------------------------------
template <bool H>
LOOM_DEV void mfma_agpr(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (H)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same MFMA with one LDS-DMA load (global_load_lds_dwordx4, scalar base
// + per-lane 32-bit byte offset, 16 bytes per lane to lds + 16 lane) folded
// around it: M0 is written before the MFMA, which supplies the wait state
// M0 needs before the load reads it.
template <bool H>
LOOM_DEV void mfma_agpr_dma(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b, uint32_t lds,
                            uint32_t voff, const void* sbase) {
  if constexpr (H)
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "v_mfma_f32_16x16x32_f16 %0, %1, %2, %0\n\t"
        "global_load_lds_dwordx4 %4, %5"
        : "+a"(acc)
        : "v"(a), "v"(b), "s"(lds), "v"(voff), "s"(sbase)
        : "memory", "m0");
  else
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n\t"
        "global_load_lds_dwordx4 %4, %5"
        : "+a"(acc)
        : "v"(a), "v"(b), "s"(lds), "v"(voff), "s"(sbase)
        : "memory", "m0");
}
// The two MFMA forms above starting a fresh accumulator (srcC = 0): the previous
// contents of acc are neither read nor needed.
template <bool H>
LOOM_DEV void mfma_agpr_z(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (H)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}
template <bool H>
LOOM_DEV void mfma_agpr_dma_z(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b, uint32_t lds,
                              uint32_t voff, const void* sbase) {
  if constexpr (H)
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "v_mfma_f32_16x16x32_f16 %0, %1, %2, 0\n\t"
        "global_load_lds_dwordx4 %4, %5"
        : "=a"(acc)
        : "v"(a), "v"(b), "s"(lds), "v"(voff), "s"(sbase)
        : "memory", "m0");
  else
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0\n\t"
        "global_load_lds_dwordx4 %4, %5"
        : "=a"(acc)
        : "v"(a), "v"(b), "s"(lds), "v"(voff), "s"(sbase)
        : "memory", "m0");
}
// LDS-DMA load with a scalar base and a per-lane 32-bit byte offset
LOOM_DEV void dma_load16_s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory", "m0");
}
// 48 wait states: every MFMA issued before has written its result
LOOM_DEV void mfma_drain() { asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory"); }

// Store of a final output that this kernel never reads back: non-temporal,
// so the written lines do not displace operands that other workgroups of the
// same XCD still read through L2 (a GEMM's C tiles would otherwise fill every
// L2 at each tile boundary and slow the K steps that follow).  Meant for
// whole-line writes: 8-byte pieces of lines stored this way measured slower.
template <class V>
LOOM_DEV void store_stream(V* p, const V& v) {
  __builtin_nontemporal_store(v, p);
}

// s_waitcnt vmcnt(n), leaving LDS and export counters alone
#define LOOM_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | ((((n) >> 4) & 3) << 14) | 0x0F70)
// s_waitcnt lgkmcnt(0): this wave's LDS reads and writes have completed
#define LOOM_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Workgroup barrier without the memory fence __syncthreads() adds (the fence
// would force every outstanding load, LDS DMA included, to complete).  The
// empty asm keeps the compiler from moving memory accesses across it.
// Compiler-only ordering of one wave's LDS accesses through pointers of
// different types (type-based alias analysis would otherwise let a read move
// above a write to the same bytes); the hardware executes a wave's LDS
// instructions in order, so no wait is needed.
LOOM_DEV void lds_order() { asm volatile("" ::: "memory"); }

LOOM_DEV void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
