// gemm.hip -- bf16 GEMM family on gfx950 MFMA: @matmul, @batch_matmul and
// @split_k_matmul_gather (the K-slab GEMM plus its fp32 gather-reduce).
//
// Reference semantics (all three accumulate sum_k x[i,k] * y[k,j]):
//   @matmul                 examples/mm/IR/00_from_helion_frontend.mlir:2-35
//   @batch_matmul           examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4-44
//   @split_k_matmul_gather  examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2-56
// Operands are row-major: A [M,K], B [K,N], C [M,N] (per batch for bmm).
//
// Kernels, fastest first (launch_gemm picks the first whose conditions hold):
//   gemm_persist_kernel  256x256 tiles, bf16 out, whole tiles dividing evenly
//                        over one workgroup per CU (>= 2 each): persistent,
//                        one LDS-DMA stream across tiles, C staged through LDS
//                        and stored as whole rows.
//   gemm_pipe_kernel<T>  T x T tiles (256, 128, 64), one per workgroup,
//                        software-pipelined LDS-DMA stages with the MFMA
//                        fragments of the next stage read during this one.
//   gemm_dma_kernel      256x256 tiles, LDS-DMA stages, K a multiple of 32.
//   gemm_bf16_kernel     any shape: register-staged 64-deep tiles (half of the
//                        threads copy A rows, the other half copy 8x8 blocks of
//                        B, transpose them in registers and store B^T), LDS rows
//                        of 128 bytes XOR-swizzled by (row & 7).
// All compute C^T tiles with v_mfma_f32_16x16x32_bf16 (B^T as the row
// operand, A^T as the column operand), fp32 accumulate, the grid flattened
// over (z, tile) with z = batch (bmm) or K-slab (split-K) and remapped so
// each XCD owns a contiguous range of tiles.
#include "common.h"

#include <atomic>
#include <type_traits>

namespace {

constexpr int kBK = 64;  // K depth of one LDS stage (8 chunks of 8 bf16)

struct GemmParams {
  const uint16_t* A;
  const uint16_t* B;
  void* C;
  int64_t M, N;
  int64_t lda, ldb, ldc;
  int64_t za, zb, zc;   // element offsets per z step for A, B, C
  int64_t k_total;      // K extent
  int64_t k_slab;       // split: K range of slab z; otherwise == k_total
  int split;            // 1: z is the K-slab index, 0: z is a batch index
  int tiles_m, tiles_n, nz;
};

template <int BM, int BN, int WM, int WN, bool ALIGNED, bool OUT_F32, bool H>
__global__ void __launch_bounds__(64 * WM * WN) gemm_bf16_kernel(GemmParams p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int HALF = NT / 2;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int CPR = kBK / 8;                     // 16-byte chunks per LDS row
  constexpr int A_PER = BM * CPR / HALF;           // A chunks per A-loading thread
  static_assert(A_PER * HALF == BM * CPR, "A tile must split evenly");
  static_assert((BN / 8) * CPR == HALF, "one 8x8 B block per B-loading thread");
  static_assert(A_PER == 8, "staging registers sized for eight 16-byte loads");
  constexpr int A_UNITS = BM * CPR, B_UNITS = BN * CPR;
  constexpr int STAGE = A_UNITS + B_UNITS;
  __shared__ u32x4_t lds[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  // ---- which tile, which z
  const int nblocks = p.tiles_m * p.tiles_n * p.nz;
  const int bid = xcd_remap(blockIdx.x, nblocks);
  const int per_z = p.tiles_m * p.tiles_n;
  const int z = bid / per_z;
  int t = bid - z * per_z;
  constexpr int GM = 8;  // tile rows per L2 group
  const int group = t / (GM * p.tiles_n);
  const int first_m = group * GM;
  const int gsz = min(p.tiles_m - first_m, GM);
  const int tin = t - group * GM * p.tiles_n;
  const int tm_idx = first_m + tin % gsz;
  const int tn_idx = tin / gsz;
  const int64_t m0 = (int64_t)tm_idx * BM, n0 = (int64_t)tn_idx * BN;

  const uint16_t* __restrict__ A = p.A;
  const uint16_t* __restrict__ B = p.B;
  int64_t kb = 0, ke = p.k_total;
  int64_t coff = (int64_t)z * p.zc;
  if (p.split) {
    kb = (int64_t)z * p.k_slab;
    ke = min(p.k_total, kb + p.k_slab);
  } else {
    A += (int64_t)z * p.za;
    B += (int64_t)z * p.zb;
  }
  const int M = (int)p.M, N = (int)p.N;

  // ---- loader roles
  const bool a_loader = tid < HALF;
  const int lt = a_loader ? tid : tid - HALF;
  // B block coordinates: k-chunk fastest so a store instruction's lanes
  // cover distinct swizzled chunks
  const int b_kc = lt % CPR, b_nc = lt / CPR;

  u32x4_t regs[8];

  auto load_tile = [&](int64_t k0) {
    if (a_loader) {
#pragma unroll
      for (int i = 0; i < A_PER; ++i) {
        const int c = lt + i * HALF;
        const int row = c / CPR, kc = c % CPR;
        const int64_t gm = m0 + row, gk = k0 + kc * 8;
        if constexpr (ALIGNED) {
          if (gm < M && gk < ke)
            regs[i] = *reinterpret_cast<const u32x4_t*>(A + gm * p.lda + gk);
          else
            regs[i] = u32x4_t{0u, 0u, 0u, 0u};
        } else {
          uint32_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            h[e] = (gm < M && gk + e < ke) ? (uint32_t)A[gm * p.lda + gk + e] : 0u;
          regs[i] = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                            h[6] | (h[7] << 16)};
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int64_t gk = k0 + b_kc * 8 + r, gn = n0 + b_nc * 8;
        if constexpr (ALIGNED) {
          if (gk < ke && gn < N)
            regs[r] = *reinterpret_cast<const u32x4_t*>(B + gk * p.ldb + gn);
          else
            regs[r] = u32x4_t{0u, 0u, 0u, 0u};
        } else {
          uint32_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            h[e] = (gk < ke && gn + e < N) ? (uint32_t)B[gk * p.ldb + gn + e] : 0u;
          regs[r] = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                            h[6] | (h[7] << 16)};
        }
      }
    }
  };

  auto store_tile = [&](int stage) {
    u32x4_t* s = lds + stage * STAGE;
    if (a_loader) {
#pragma unroll
      for (int i = 0; i < A_PER; ++i) {
        const int c = lt + i * HALF;
        const int row = c / CPR, kc = c % CPR;
        s[row * CPR + (kc ^ (row & 7))] = regs[i];
      }
    } else {
      u32x4_t tr[8];
      transpose8x8(regs, tr);
      u32x4_t* sb = s + A_UNITS;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = b_nc * 8 + j;  // n & 7 == j
        sb[n * CPR + (b_kc ^ j)] = tr[j];
      }
    }
  };

  const int wm = wave % WM, wn = wave / WM;
  const int lrow = lane & 15, lgrp = lane >> 4;
  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage) {
    const u32x4_t* sa = lds + stage * STAGE;
    const u32x4_t* sb = sa + A_UNITS;
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      u32x4_t af[TM], bfr[TN];
      const int ch = ks * 4 + lgrp;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WTM + i * 16 + lrow;
        af[i] = sa[row * CPR + (ch ^ (row & 7))];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = wn * WTN + j * 16 + lrow;
        bfr[j] = sb[n * CPR + (ch ^ (n & 7))];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16t<H>(af[i], bfr[j], acc[i][j]);
    }
  };

  const int64_t nk = ke > kb ? (ke - kb + kBK - 1) / kBK : 0;
  if (nk > 0) {
    load_tile(kb);
    store_tile(0);
  }
  __syncthreads();
  for (int64_t it = 0; it < nk; ++it) {
    if (it + 1 < nk) load_tile(kb + (it + 1) * kBK);
    compute((int)(it & 1));
    if (it + 1 < nk) store_tile((int)((it + 1) & 1));
    __syncthreads();
  }

  // ---- epilogue: accumulator row 4*(lane/16)+r, column lane%16
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * WTN + j * 16 + lrow;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * WTM + i * 16 + lgrp * 4 + r;
        if (row < M && col < N) {
          if constexpr (OUT_F32)
            static_cast<float*>(p.C)[coff + row * p.ldc + col] = acc[i][j][r];
          else
            static_cast<uint16_t*>(p.C)[coff + row * p.ldc + col] = (uint16_t)cvt16<H>(acc[i][j][r]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 256x256 tile, LDS-DMA pipeline.  Four waves, each owning a 128x128 block of
// C.  Per stage, A [256][BK] and B [BK][256] are copied global -> LDS by
// global_load_lds_dwordx4 (no staging registers; addresses clamped inside
// each operand, the rows and columns past its extent are never stored),
// NS stages deep.  B stays in its [k][n] layout: the MFMA
// operand with eight consecutive k per lane comes from two ds_read_b64_tr_b16.
// The MFMA computes C^T tiles (B^T as the row operand, A^T as the column
// operand), so each lane ends with four consecutive columns of one row of C:
// 8-byte (bf16) or 16-byte (fp32) stores straight from registers.
// Swizzles (16-byte chunk index XOR a function of the row, a_swz / b_swz)
// keep the operand reads free of bank conflicts; the DMA writes are linear
// 1 KB blocks per instruction.
// Each stage buffer is its own __shared__ array and the main loop is unrolled
// by NS, so every LDS address is a constant offset; the DMAs are issued from
// inline assembly and waited for by hand (s_waitcnt vmcnt(n) for the stage
// needed next), with barriers that do not drain the DMAs still in flight.
// ---------------------------------------------------------------------------
// gfx950's LDS has 128 four-byte banks (512 bytes) and serves a wave's
// ds_read_b128 / ds_read_b64_tr_b16 in two passes of 32 lanes, so the 32
// lanes of one pass must touch 32 distinct 16-byte slots of a 512-byte window
// (measured: the bank-conflict counter reads zero for linear addresses and
// one conflict cycle per pass when two lanes share a slot).
// A rows hold BK/8 16-byte chunks; a fragment read covers 16 consecutive rows
// and two chunk columns per pass.  BK 32 (64-byte rows): rows r and r ^ 8
// share a window position, so bit 3 of the row flips chunk bit 1.  BK 64
// (128-byte rows): rows r, r ^ 4, r ^ 8, r ^ 12 share one, so row bits 2-3
// pick the chunk pair.
template <int BK>
LOOM_DEV int a_swz(int row) {
  if constexpr (BK == 64)
    return 2 * ((row >> 2) & 3);
  else
    return 2 * ((row >> 3) & 1);
}
// B rows hold 32 chunks; one pass of a transposed read covers k rows k..k+3
// and k+8..k+11, 32 bytes each (T 256: 512-byte rows, all at one window
// position; T 128: 256-byte rows, alternating halves): 2 (k & 3) and
// 8 ((k >> 3) & 1) put the eight pieces in distinct 32-byte slots.
LOOM_DEV int b_swz(int k) { return (2 * (k & 3)) ^ (8 * ((k >> 3) & 1)); }

template <int BK, int NS, bool OUT_F32, bool H>
__global__ void __launch_bounds__(256) gemm_dma_kernel(GemmParams p) {
  constexpr int BM = 256, BN = 256;
  constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
  constexpr int A_ROWS_PER_I = 1024 / (BK * 2);   // A rows per DMA instruction
  constexpr int A_CPR = BK / 8;                   // 16-byte chunks per A row
  constexpr int A_INSTR = A_BYTES / 1024 / 4;     // per wave per stage
  constexpr int B_INSTR = B_BYTES / 1024 / 4;
  constexpr int LPW = A_INSTR + B_INSTR;          // DMA instructions per wave per stage
  static_assert(NS >= 2 && NS <= 4, "2..4 stages");
  static_assert(LPW * (NS - 2) <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char sA0[A_BYTES], sB0[B_BYTES];
  __shared__ __attribute__((aligned(1024))) char sA1[A_BYTES], sB1[B_BYTES];
  __shared__ __attribute__((aligned(1024))) char sA2[NS > 2 ? A_BYTES : 16], sB2[NS > 2 ? B_BYTES : 16];
  __shared__ __attribute__((aligned(1024))) char sA3[NS > 3 ? A_BYTES : 16], sB3[NS > 3 ? B_BYTES : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform by construction; readfirstlane lets the compiler know (the
  // LDS destination of a DMA load lives in M0)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- which tile, which z (XCD-contiguous, grouped by 8 tile rows)
  const int nblocks = p.tiles_m * p.tiles_n * p.nz;
  const int bid = xcd_remap(blockIdx.x, nblocks);
  const int per_z = p.tiles_m * p.tiles_n;
  const int z = bid / per_z;
  const int t = bid - z * per_z;
  constexpr int GM = 8;
  const int group = t / (GM * p.tiles_n);
  const int first_m = group * GM;
  const int gsz = min(p.tiles_m - first_m, GM);
  const int tin = t - group * GM * p.tiles_n;
  const int64_t m0 = (int64_t)(first_m + tin % gsz) * BM;
  const int64_t n0 = (int64_t)(tin / gsz) * BN;

  const uint16_t* A = p.A;
  const uint16_t* B = p.B;
  int64_t kb = 0, ke = p.k_total;
  if (p.split) {
    kb = (int64_t)z * p.k_slab;
    ke = min(p.k_total, kb + p.k_slab);
  } else {
    A += (int64_t)z * p.za;
    B += (int64_t)z * p.zb;
  }

  auto stageA = [&](int s) -> lds_char_t* {
    if (s == 0) return (lds_char_t*)sA0;
    if (s == 1) return (lds_char_t*)sA1;
    if (s == 2) return (lds_char_t*)sA2;
    return (lds_char_t*)sA3;
  };
  auto stageB = [&](int s) -> lds_char_t* {
    if (s == 0) return (lds_char_t*)sB0;
    if (s == 1) return (lds_char_t*)sB1;
    if (s == 2) return (lds_char_t*)sB2;
    return (lds_char_t*)sB3;
  };

  // ---- DMA one stage: this wave's A_INSTR + B_INSTR 1 KB blocks
  auto issue = [&](int s, int64_t k0) {
    const uint32_t la = lds_addr(stageA(s));
    const uint32_t lb = lds_addr(stageB(s));
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const int j = wave * A_INSTR + i;
      const int row = j * A_ROWS_PER_I + lane / A_CPR;
      const int c = (lane % A_CPR) ^ a_swz<BK>(row);
      const int64_t gm = min<int64_t>(m0 + row, p.M - 1);
      dma_load16(A + gm * p.lda + k0 + c * 8, la + j * 1024);
    }
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
      const int j = wave * B_INSTR + i;
      const int row = j * 2 + lane / 32;
      const int c = (lane % 32) ^ b_swz(row);
      const int64_t gn = min<int64_t>(n0 + c * 8, p.N - 8);
      dma_load16(B + (k0 + row) * p.ldb + gn, lb + j * 1024);
    }
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;
  f32x4_t acc[8][8];  // [n tile][m tile]
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s) {
    const lds_char_t* la = stageA(s);
    const lds_char_t* lb = stageB(s);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      u32x4_t af[8];
#pragma unroll
      for (int tm = 0; tm < 8; ++tm) {
        // column operand A^T: lane holds A[m][32 ks + 8 lg .. +7], m = tile row lr
        const int m = wm * 128 + tm * 16 + lr;
        const int ch = (ks * 4 + lg) ^ a_swz<BK>(m);
        af[tm] = *(const __attribute__((address_space(3))) u32x4_t*)(la + m * (BK * 2) + ch * 16);
      }
#pragma unroll
      for (int tn = 0; tn < 8; ++tn) {
        // row operand B^T: lane holds B[32 ks + 8 lg .. +7][n], n = tile col lr
        const int nb = wn * 128 + tn * 16;
        const int a = lr >> 2, c4 = lr & 3;
        const int k0r = ks * 32 + lg * 8 + a;          // & 3 == a
        const int ch = ((nb >> 3) + (c4 >> 1)) ^ b_swz(k0r);
        const lds_char_t* q = lb + k0r * 512 + ch * 16 + (c4 & 1) * 8;
        const u32x2_t lo = lds_read_tr16(q);
        const u32x2_t hi = lds_read_tr16(q + 4 * 512);
        const u32x4_t bf = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int tm = 0; tm < 8; ++tm) acc[tn][tm] = mfma16t<H>(bf, af[tm], acc[tn][tm]);
      }
    }
  };

  const int nk = ke > kb ? (int)((ke - kb) / BK) : 0;  // K range is a multiple of BK
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s, kb + (int64_t)s * BK);

  for (int it0 = 0; it0 < nk; it0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int it = it0 + s;
      if (it < nk) {
        // my DMA for stage `it` is done once at most the younger stages'
        // loads are outstanding; the barrier makes everyone's visible and
        // frees the buffer read in the previous iteration
        const int younger = min(NS - 2, nk - 1 - it);
        if (younger >= 2) LOOM_WAIT_VMCNT(2 * LPW);
        else if (younger == 1) LOOM_WAIT_VMCNT(LPW);
        else LOOM_WAIT_VMCNT(0);
        barrier_nofence();
        if (it + NS - 1 < nk) issue((s + NS - 1) % NS, kb + (int64_t)(it + NS - 1) * BK);
        compute(s);
      }
    }
  }

  // ---- epilogue: acc[tn][tm][i] = C[m][n + i], m = tile row, n = 4 lg.
  // The scheduling fences keep the compiler from pulling all 256 accumulators
  // into VGPRs at once (which would set the kernel's VGPR budget).
#pragma unroll
  for (int tm = 0; tm < 8; ++tm) {
    __builtin_amdgcn_sched_barrier(0);
    const int64_t row = m0 + wm * 128 + tm * 16 + lr;
    if (row >= p.M) continue;
#pragma unroll
    for (int tn = 0; tn < 8; ++tn) {
      const int64_t col = n0 + wn * 128 + tn * 16 + lg * 4;
      if (col >= p.N) continue;
      const f32x4_t v = acc[tn][tm];
      if constexpr (OUT_F32)
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.C) + (int64_t)z * p.zc + row * p.ldc + col) = v;
      else
        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.C) + (int64_t)z * p.zc + row * p.ldc + col) =
            u32x2_t{pack2<H>(v[0], v[1]), pack2<H>(v[2], v[3])};
    }
  }
}

// ---------------------------------------------------------------------------
// Square T x T tile (T = 256, 128 or 64), software-pipelined: the production path
// for K ranges that are whole multiples of NS*BK.  Four waves, each owning a
// (T/2) x (T/2) block of C^T tiles; A [T][32] and B [32][T] stages arrive by
// LDS DMA, NS deep (T 256: 4 stages of 32 KB; 128: 4 of 16 KB; 64: 8 of
// 8 KB).  Deeper rings of the smaller tiles (8 and 16 stages, 128 KB) were
// slower: split-K 512x512x16384 23.9 against 23.0 us, mm 1024^3 from HBM 8.0
// against 7.6 us (4 and 2 stages: 31.9 us and 8.1 us).
// The LDS layouts, swizzles and operand roles are those of gemm_dma_kernel
// (and the accumulation order too: results are bitwise identical); what
// differs is the schedule:
//   - the MFMA fragments of stage it+1 are read from LDS into a second
//     register set while the MFMAs of stage it run, spread between them;
//   - this wave's DMA for stage it+NS is folded between the MFMAs too (one
//     per group of T/32 MFMAs), with a scalar base per stage and per-lane
//     32-bit offsets that stay the same for every stage;
//   - the accumulators live in AGPRs (inline-asm MFMAs, see mfma_agpr) and
//     the loop body has no data-dependent branch: past the last stage the
//     DMA re-reads the last stage into a buffer that is never read again;
//   - full tiles convert every accumulator first and then store without
//     bounds checks.
// One barrier per stage: it publishes stage it+1 (everyone's DMA landed,
// each wave having waited for its own) and, because every wave waited for
// its fragment reads of stage it before it, frees stage it's buffer for the
// DMA of stage it+NS.
// ---------------------------------------------------------------------------
// Orders every later read of the accumulators after the preceding
// mfma_drain(): the MFMAs are inline assembly, so nothing else tells the
// compiler that the drain must come first.
template <int TT>
LOOM_DEV void acc_fence(f32x4_t (&acc)[TT][TT]) {
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) asm volatile("" : "+a"(acc[i][j]));
}

template <int T>
constexpr int pipe_stages() { return T == 256 ? 4 : T == 128 ? 4 : 8; }

// B swizzle of the pipelined kernels.  Rows of 256 bytes or more: b_swz.
// T = 64 has 128-byte rows (8 chunks): rows k..k+3 of one pass already sit at
// four window positions and rows k+8..k+11 repeat them, so bit 3 of the row
// flips chunk bit 1 instead.
template <int T>
LOOM_DEV int b_swz_t(int k) {
  if constexpr (T == 64)
    return (2 * (k & 3)) ^ (2 * ((k >> 3) & 1));
  else
    return b_swz(k);
}

template <int T, bool OUT_F32, bool H>
__global__ void __launch_bounds__(256) gemm_pipe_kernel(GemmParams p) {
  constexpr int NS = pipe_stages<T>(), BK = 32;
  constexpr int TT = T / 32;                     // 16-wide tiles per wave dimension
  constexpr int A_BYTES = T * BK * 2, B_BYTES = BK * T * 2;
  constexpr int B_ROW = T * 2;                   // bytes per B row in LDS
  constexpr int A_INSTR = A_BYTES / 1024 / 4;    // DMA instructions per wave per stage
  constexpr int B_INSTR = B_BYTES / 1024 / 4;
  constexpr int LPW = A_INSTR + B_INSTR;
  constexpr int B_RPI = 1024 / B_ROW, B_CPR = B_ROW / 16;   // B rows per DMA, chunks per row
  static_assert(T == 256 || T == 128 || T == 64, "tile");
  static_assert(LPW == TT, "one DMA per group of TT MFMAs");
  static_assert(NS % 2 == 0 && (NS - 1) * LPW <= 63, "stages");
  __shared__ __attribute__((aligned(1024))) char smem[NS * (A_BYTES + B_BYTES)];
  lds_char_t* const lds = (lds_char_t*)smem;
  auto stageA = [&](int s) { return lds + s * A_BYTES; };
  auto stageB = [&](int s) { return lds + NS * A_BYTES + s * B_BYTES; };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // ---- which tile, which z (XCD-contiguous, grouped by 8 tile rows)
  const int nblocks = p.tiles_m * p.tiles_n * p.nz;
  const int bid = xcd_remap(blockIdx.x, nblocks);
  const int per_z = p.tiles_m * p.tiles_n;
  const int z = bid / per_z;
  const int t = bid - z * per_z;
  constexpr int GM = 8;
  const int group = t / (GM * p.tiles_n);
  const int first_m = group * GM;
  const int gsz = min(p.tiles_m - first_m, GM);
  const int tin = t - group * GM * p.tiles_n;
  const int64_t m0 = (int64_t)(first_m + tin % gsz) * T;
  const int64_t n0 = (int64_t)(tin / gsz) * T;

  const uint16_t* A = p.A;
  const uint16_t* B = p.B;
  int64_t kb = 0, ke = p.k_total;
  if (p.split) {
    kb = (int64_t)z * p.k_slab;
    ke = min(p.k_total, kb + p.k_slab);
  } else {
    A += (int64_t)z * p.za;
    B += (int64_t)z * p.zb;
  }
  const int nk = (int)((ke - kb) / BK);   // the host guarantees nk % NS == 0, nk >= NS

  // ---- per-lane DMA byte offsets (rows / columns past the operand clamped
  // inside it; what they load is never stored)
  uint32_t aoff[A_INSTR], boff[B_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int row = (wave * A_INSTR + i) * 16 + lane / 4;
    const int64_t gm = min<int64_t>(row, p.M - 1 - m0);
    aoff[i] = (uint32_t)(gm * p.lda * 2 + ((lane % 4) ^ a_swz<BK>(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int row = (wave * B_INSTR + i) * B_RPI + lane / B_CPR;
    const int64_t gn = min<int64_t>(((lane % B_CPR) ^ b_swz_t<T>(row)) * 8, p.N - 8 - n0);
    boff[i] = (uint32_t)(row * p.ldb * 2 + gn * 2);
  }
  const uint16_t* const Abase = A + m0 * p.lda + kb;
  const uint16_t* const Bbase = B + n0 + kb * p.ldb;
  const uint32_t la0 = lds_addr(stageA(0)), lb0 = lds_addr(stageB(0));
  auto issue = [&](int s, int stage) {
    const uint16_t* ab = Abase + (int64_t)stage * BK;
    const uint16_t* bb = Bbase + (int64_t)stage * BK * p.ldb;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      dma_load16_s(aoff[i], ab, la0 + s * A_BYTES + (wave * A_INSTR + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i)
      dma_load16_s(boff[i], bb, lb0 + s * B_BYTES + (wave * B_INSTR + i) * 1024);
  };

  // ---- fragment addresses.  A: one lane offset (tile tm moves by 1 KB; the
  // swizzle depends on the row's low four bits only).  B: the 16-byte chunk
  // of tile tn is ((T/16) wn | 2 tn | c4 >> 1) ^ swizzle, i.e. the lane
  // offset XOR (tn << 5).  Stage bases are immediate offsets.
  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t a_lane = (uint32_t)((wm * (T / 2) + lr) * (BK * 2) + ((lg ^ a_swz<BK>(lr)) * 16));
  uint32_t b_lane[TT];
  {
    const int a = lr >> 2, c4 = lr & 3;
    const int k0r = lg * 8 + a;
    const uint32_t base = (uint32_t)(k0r * B_ROW + (((wn * (T / 16)) | (c4 >> 1)) ^ b_swz_t<T>(k0r)) * 16 +
                                     (c4 & 1) * 8);
#pragma unroll
    for (int tn = 0; tn < TT; ++tn) b_lane[tn] = base ^ (uint32_t)(tn << 5);
  }
  auto read_a = [&](int s, int tm) {
    return *(const __attribute__((address_space(3))) u32x4_t*)(stageA(s) + a_lane + tm * 1024);
  };
  auto read_b = [&](int s, int tn, int half) {
    return lds_read_tr16(stageB(s) + b_lane[tn] + half * 4 * B_ROW);
  };

  f32x4_t acc[TT][TT];  // [n tile][m tile]: C^T tiles
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // the zeros above are written by ordinary instructions; the first
  // inline-asm MFMA that reads them as srcC needs them retired
  mfma_drain();

  // ---- prologue: NS stages in flight, fragments of stage 0
  u32x4_t af[2][TT], bfr[2][TT];
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(s, s);
  LOOM_WAIT_VMCNT((NS - 1) * LPW);
  barrier_nofence();
#pragma unroll
  for (int q = 0; q < TT; ++q) {
    af[0][q] = read_a(0, q);
    const u32x2_t lo = read_b(0, q, 0), hi = read_b(0, q, 1);
    bfr[0][q] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
  }

  // ---- one stage: TT*TT MFMAs on the current set; per group of TT (tile
  // tn): the next set's B fragment tn (two transposed reads) and A fragment
  // tn, and this wave's DMA number tn for stage it+NS
  auto step = [&](int u, int it, const u32x4_t (&fa)[TT], const u32x4_t (&fb)[TT],
                  u32x4_t (&na)[TT], u32x4_t (&nb)[TT]) {
    LOOM_WAIT_VMCNT((NS - 2) * LPW);
    LOOM_WAIT_LGKM0();
    barrier_nofence();
    const int sn = (u + 1) % NS;
    const int sd = min(it + NS, nk - 1);
    const uint16_t* ab = Abase + (int64_t)sd * BK;
    const uint16_t* bb = Bbase + (int64_t)sd * BK * p.ldb;
    u32x2_t lo[TT];
#pragma unroll
    for (int i = 0; i < TT * TT; ++i) {
      const int tn = i / TT, tm = i % TT;
      if (tm == TT / 2) {
        if (tn < A_INSTR)
          mfma_agpr_dma<H>(acc[tn][tm], fb[tn], fa[tm],
                           la0 + (u % NS) * A_BYTES + (wave * A_INSTR + tn) * 1024, aoff[tn], ab);
        else
          mfma_agpr_dma<H>(acc[tn][tm], fb[tn], fa[tm],
                           lb0 + (u % NS) * B_BYTES + (wave * B_INSTR + tn - A_INSTR) * 1024,
                           boff[tn - A_INSTR], bb);
      } else {
        mfma_agpr<H>(acc[tn][tm], fb[tn], fa[tm]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (tm == 0) lo[tn] = read_b(sn, tn, 0);
      if (tm == TT / 4) {
        const u32x2_t hi = read_b(sn, tn, 1);
        nb[tn] = u32x4_t{lo[tn][0], lo[tn][1], hi[0], hi[1]};
      }
      if (tm == 3 * TT / 4) na[tn] = read_a(sn, tn);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int it0 = 0; it0 < nk; it0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u)
      step(u, it0 + u, af[u & 1], bfr[u & 1], af[(u & 1) ^ 1], bfr[(u & 1) ^ 1]);
  }
  LOOM_WAIT_VMCNT(0);   // the trailing re-reads land before the workgroup ends
  // every MFMA has written its accumulator before the epilogue reads them
  // (acc_fence keeps those reads after the drain)
  mfma_drain();
  acc_fence(acc);

  // ---- epilogue: acc[tn][tm][i] = C[m][n + i], m = tile row lr, n = 4 lg
  void* const cz = OUT_F32 ? (void*)(static_cast<float*>(p.C) + (int64_t)z * p.zc)
                           : (void*)(static_cast<uint16_t*>(p.C) + (int64_t)z * p.zc);
  const int64_t r0 = m0 + wm * (T / 2) + lr, c0 = n0 + wn * (T / 2) + lg * 4;
  // Full tiles whose C fits the stage ring (all but fp32 at T 256) are
  // staged there row-major and stored as whole rows, 16 bytes per lane:
  // the register layout gives each lane 16-byte (fp32) or 8-byte (bf16)
  // pieces of 16 rows per store, which reach memory as partial lines.  Chunk
  // c of row rr sits at position c ^ c_swz(rr): each pass of the staging
  // writes (16 rows, one 16-byte chunk of each: 16 lanes of 16 bytes, or 32
  // of 8) then covers the 64 banks (a 256-byte window) once.
  constexpr int ES = OUT_F32 ? 4 : 2, CRB = T * ES, CNC = CRB / 16;
  constexpr bool STAGED_C = T * CRB <= NS * (A_BYTES + B_BYTES);
  constexpr int CRPW = CRB >= 256 ? 1 : 256 / CRB;         // rows per 256-byte bank window
  constexpr int CSWM = (CNC < 16 ? CNC : 16) - 1;
  auto c_swz = [](int rr) { return (rr / CRPW) & CSWM; };
  if constexpr (STAGED_C) {
    if (m0 + T <= p.M && n0 + T <= p.N) {
      LOOM_WAIT_LGKM0();      // this wave's last fragment reads; every wave's DMAs
      barrier_nofence();      // landed (vmcnt 0 above): the ring is free
#pragma unroll
      for (int tm = 0; tm < TT; ++tm) {
        const int rr = wm * (T / 2) + tm * 16 + lr;
#pragma unroll
        for (int tn = 0; tn < TT; ++tn) {
          const int col = wn * (T / 2) + tn * 16 + lg * 4;
          const int cpos = ((col * ES) / 16) ^ c_swz(rr);
          lds_char_t* const dst = lds + rr * CRB + cpos * 16 + (col * ES) % 16;
          if constexpr (OUT_F32)
            *reinterpret_cast<__attribute__((address_space(3))) f32x4_t*>(dst) = acc[tn][tm];
          else
            *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(dst) =
                u32x2_t{pack2<H>(acc[tn][tm][0], acc[tn][tm][1]),
                        pack2<H>(acc[tn][tm][2], acc[tn][tm][3])};
        }
      }
      LOOM_WAIT_LGKM0();
      barrier_nofence();
      char* const cbase = static_cast<char*>(cz) + (m0 * p.ldc + n0) * ES;
#pragma unroll
      for (int k = 0; k < T * CNC / 4 / 64; ++k) {     // wave w: rows w T/4 .. (w+1) T/4 - 1
        const int idx = (wave * (T / 4)) * CNC + k * 64 + lane;
        const int rr = idx / CNC, cp = idx % CNC;
        const u32x4_t v =
            *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(lds + idx * 16);
        *reinterpret_cast<u32x4_t*>(cbase + (int64_t)rr * p.ldc * ES + (cp ^ c_swz(rr)) * 16) = v;
      }
      return;
    }
  }
  if (m0 + T <= p.M && n0 + T <= p.N) {
    if constexpr (OUT_F32) {
      float* cb = static_cast<float*>(cz) + r0 * p.ldc + c0;
#pragma unroll
      for (int tm = 0; tm < TT; ++tm)
#pragma unroll
        for (int tn = 0; tn < TT; ++tn)
          *reinterpret_cast<f32x4_t*>(cb + (int64_t)(tm * 16) * p.ldc + tn * 16) = acc[tn][tm];
    } else {
      u32x2_t pk[TT][TT];
#pragma unroll
      for (int tn = 0; tn < TT; ++tn)
#pragma unroll
        for (int tm = 0; tm < TT; ++tm)
          pk[tn][tm] = u32x2_t{pack2<H>(acc[tn][tm][0], acc[tn][tm][1]),
                               pack2<H>(acc[tn][tm][2], acc[tn][tm][3])};
      uint16_t* cb = static_cast<uint16_t*>(cz) + r0 * p.ldc + c0;
#pragma unroll
      for (int tm = 0; tm < TT; ++tm)
#pragma unroll
        for (int tn = 0; tn < TT; ++tn)
          *reinterpret_cast<u32x2_t*>(cb + (int64_t)(tm * 16) * p.ldc + tn * 16) = pk[tn][tm];
    }
    return;
  }
#pragma unroll
  for (int tm = 0; tm < TT; ++tm) {
    __builtin_amdgcn_sched_barrier(0);
    const int64_t row = r0 + tm * 16;
    if (row >= p.M) continue;
#pragma unroll
    for (int tn = 0; tn < TT; ++tn) {
      const int64_t col = c0 + tn * 16;
      if (col >= p.N) continue;
      const f32x4_t v = acc[tn][tm];
      if constexpr (OUT_F32)
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(cz) + row * p.ldc + col) = v;
      else
        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(cz) + row * p.ldc + col) =
            u32x2_t{pack2<H>(v[0], v[1]), pack2<H>(v[2], v[3])};
    }
  }
}

// Launches the pipelined kernel when every K range is a whole number of its
// NS*32-deep rounds (and the per-lane DMA offsets fit in 32 bits).
template <int T, bool H>
bool launch_pipe(const GemmParams& p, bool aligned, bool out_f32, hipStream_t st) {
  constexpr int round = pipe_stages<T>() * 32;
  const bool ok = aligned && p.k_total % round == 0 && (!p.split || p.k_slab % round == 0) &&
                  p.lda < (1 << 22) && p.ldb < (1 << 22) && p.N >= 8;
  if (!ok) return false;
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n * p.nz)), block(256);
  if (out_f32)
    hipLaunchKernelGGL((gemm_pipe_kernel<T, true, H>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((gemm_pipe_kernel<T, false, H>), grid, block, 0, st, p);
  return true;
}

// ---------------------------------------------------------------------------
// Persistent 256x256 GEMM (bf16 output, whole tiles): one workgroup per CU
// walks nr tiles with one continuous LDS-DMA stream, so the first stages of
// tile r+1 load while tile r finishes, and no workgroup launch, set-up or
// cold pipeline separates the tiles.  Workgroup g (on XCD g % 8) runs the
// tiles that the one-tile-per-workgroup launch would run on that XCD, in the
// same rounds: logical tile (g % 8) ntiles/8 + r G/8 + g / 8.
//
// Stage slots hold A and B of one 32-deep K step (slot = global step % 4),
// and a fifth 32 KB region stages C: each tile's epilogue converts the
// accumulators to bf16 a quarter (two 16-row groups per wave) at a time,
// writes them row-major into that region (16-byte chunks XOR row & 15) and
// stores whole 512-byte rows, 16 bytes per lane.  Before the first store
// every LDS-DMA load issued so far has landed (vmcnt 0), so the stores only
// add to the count the main loop's vmcnt waits see: those waits stay exact.
// The first K step of every tile starts its accumulators with srcC = 0.
// ---------------------------------------------------------------------------
template <bool H>
__global__ void __launch_bounds__(256) gemm_persist_kernel(GemmParams p, int nr) {
  constexpr int T = 256, NS = 4, BK = 32, TT = 8;
  constexpr int A_BYTES = T * BK * 2, B_BYTES = BK * T * 2, SLOT = A_BYTES + B_BYTES;
  constexpr int B_ROW = T * 2;
  constexpr int A_INSTR = A_BYTES / 1024 / 4, B_INSTR = B_BYTES / 1024 / 4;
  constexpr int LPW = A_INSTR + B_INSTR;
  constexpr int B_RPI = 1024 / B_ROW, B_CPR = B_ROW / 16;
  constexpr int E_ROWS = 64;                          // C staging rows of 512 bytes
  static_assert(LPW == TT && NS == 4, "one DMA per group of TT MFMAs");
  __shared__ __attribute__((aligned(1024))) char smem[NS * SLOT + E_ROWS * 512];
  lds_char_t* const lds = (lds_char_t*)smem;
  lds_char_t* const cst = lds + NS * SLOT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = (int)gridDim.x;
  const int per_x = p.tiles_m * p.tiles_n * p.nz / 8;
  const int gx = (int)blockIdx.x % 8, gj = (int)blockIdx.x / 8;
  const int nk = (int)(p.k_total / BK);   // host: nk % NS == 0, nk >= NS

  auto tile_of = [&](int r, int& z, int64_t& m0, int64_t& n0) {
    const int l = gx * per_x + r * (G / 8) + gj;
    const int per_z = p.tiles_m * p.tiles_n;
    z = l / per_z;
    const int t = l - z * per_z;
    constexpr int GM = 8;
    const int group = t / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gsz = min(p.tiles_m - first_m, GM);
    const int tin = t - group * GM * p.tiles_n;
    m0 = (int64_t)(first_m + tin % gsz) * T;
    n0 = (int64_t)(tin / gsz) * T;
  };
  // A, B and C of tile r at k = 0
  auto tile_ptrs = [&](int r, const uint16_t*& a, const uint16_t*& b, char*& c) {
    int z;
    int64_t m0, n0;
    tile_of(r, z, m0, n0);
    a = p.A + (int64_t)z * p.za + m0 * p.lda;
    b = p.B + (int64_t)z * p.zb + n0;
    c = reinterpret_cast<char*>(static_cast<uint16_t*>(p.C) + (int64_t)z * p.zc + m0 * p.ldc + n0);
  };

  uint32_t aoff[A_INSTR], boff[B_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int row = (wave * A_INSTR + i) * 16 + lane / 4;
    aoff[i] = (uint32_t)(row * p.lda * 2 + ((lane % 4) ^ a_swz<BK>(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int row = (wave * B_INSTR + i) * B_RPI + lane / B_CPR;
    boff[i] = (uint32_t)(row * p.ldb * 2 + ((lane % B_CPR) ^ b_swz(row)) * 16);
  }
  const uint32_t l0 = lds_addr(lds);
  auto issue = [&](int slot, const uint16_t* ab, const uint16_t* bb) {
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      dma_load16_s(aoff[i], ab, l0 + slot * SLOT + (wave * A_INSTR + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i)
      dma_load16_s(boff[i], bb, l0 + slot * SLOT + A_BYTES + (wave * B_INSTR + i) * 1024);
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t a_lane = (uint32_t)((wm * (T / 2) + lr) * (BK * 2) + ((lg ^ a_swz<BK>(lr)) * 16));
  uint32_t b_lane[TT];
  {
    const int a = lr >> 2, c4 = lr & 3;
    const int k0r = lg * 8 + a;
    const uint32_t base =
        (uint32_t)(k0r * B_ROW + (((wn * (T / 16)) | (c4 >> 1)) ^ b_swz(k0r)) * 16 + (c4 & 1) * 8);
#pragma unroll
    for (int tn = 0; tn < TT; ++tn) b_lane[tn] = base ^ (uint32_t)(tn << 5);
  }
  auto read_a = [&](int s, int tm) {
    return *(const __attribute__((address_space(3))) u32x4_t*)(lds + s * SLOT + a_lane + tm * 1024);
  };
  auto read_b = [&](int s, int tn, int half) {
    return lds_read_tr16(lds + s * SLOT + A_BYTES + b_lane[tn] + half * 4 * B_ROW);
  };

  // per-lane byte offset of the epilogue's 16-byte stores within a tile
  const uint32_t st_lane =
      (uint32_t)((((wave >> 1) * 128 + (wave & 1) * 16 + (lane >> 5)) * p.ldc + (lane & 31) * 8) * 2);

  f32x4_t acc[TT][TT];  // [n tile][m tile]: C^T tiles; every tile's first step sets them
  u32x4_t af[2][TT], bfr[2][TT];

  // ---- prologue: K steps 0..NS-1 of tile 0, fragments of step 0
  const uint16_t *ar, *br;
  char* cr;
  tile_ptrs(0, ar, br, cr);
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(s, ar + s * BK, br + (int64_t)s * BK * p.ldb);
  LOOM_WAIT_VMCNT((NS - 1) * LPW);
  barrier_nofence();
#pragma unroll
  for (int q = 0; q < TT; ++q) {
    af[0][q] = read_a(0, q);
    const u32x2_t lo = read_b(0, q, 0), hi = read_b(0, q, 1);
    bfr[0][q] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
  }

  // ---- one K step (slot u): TT*TT MFMAs on the current fragments; per group
  // of TT (tile tn) the next step's fragments and this wave's DMA number tn of
  // global step +NS into slot u
  auto step = [&](auto firstc, int u, const uint16_t* ab, const uint16_t* bb,
                  const u32x4_t (&fa)[TT], const u32x4_t (&fb)[TT], u32x4_t (&na)[TT],
                  u32x4_t (&nb)[TT]) {
    constexpr bool FIRST = decltype(firstc)::value;
    LOOM_WAIT_VMCNT((NS - 2) * LPW);
    LOOM_WAIT_LGKM0();
    barrier_nofence();
    const int sn = (u + 1) % NS;
    u32x2_t lo[TT];
#pragma unroll
    for (int i = 0; i < TT * TT; ++i) {
      const int tn = i / TT, tm = i % TT;
      if (tm == TT / 2) {
        const uint32_t dst = tn < A_INSTR ? l0 + u * SLOT + (wave * A_INSTR + tn) * 1024
                                          : l0 + u * SLOT + A_BYTES + (wave * B_INSTR + tn - A_INSTR) * 1024;
        const uint32_t voff = tn < A_INSTR ? aoff[tn] : boff[tn - A_INSTR];
        const uint16_t* sb = tn < A_INSTR ? ab : bb;
        if constexpr (FIRST)
          mfma_agpr_dma_z<H>(acc[tn][tm], fb[tn], fa[tm], dst, voff, sb);
        else
          mfma_agpr_dma<H>(acc[tn][tm], fb[tn], fa[tm], dst, voff, sb);
      } else {
        if constexpr (FIRST)
          mfma_agpr_z<H>(acc[tn][tm], fb[tn], fa[tm]);
        else
          mfma_agpr<H>(acc[tn][tm], fb[tn], fa[tm]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (tm == 0) lo[tn] = read_b(sn, tn, 0);
      if (tm == TT / 4) {
        const u32x2_t hi = read_b(sn, tn, 1);
        nb[tn] = u32x4_t{lo[tn][0], lo[tn][1], hi[0], hi[1]};
      }
      if (tm == 3 * TT / 4) na[tn] = read_a(sn, tn);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // NS steps; the DMA of step u loads K step (ab + u sa, bb + u sb), i.e. NS
  // steps ahead: this tile's next NS steps, or in the tile's last NS steps the
  // next tile's first NS (after the last tile: the last step again, sa = sb = 0)
  auto group = [&](auto firstc, const uint16_t* ab, const uint16_t* bb, int64_t sa, int64_t sb) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      if (u == 0)
        step(firstc, u, ab, bb, af[0], bfr[0], af[1], bfr[1]);
      else
        step(std::false_type{}, u, ab + u * sa, bb + u * sb, af[u & 1], bfr[u & 1], af[(u & 1) ^ 1],
             bfr[(u & 1) ^ 1]);
    }
  };

  const int ng = nk / NS;
  for (int r = 0; r < nr; ++r) {
    const uint16_t *an, *bn;
    char* cn;
    int64_t sa = BK, sb = (int64_t)BK * p.ldb;
    if (r + 1 < nr) {
      tile_ptrs(r + 1, an, bn, cn);
    } else {
      an = ar + (nk - 1) * BK;
      bn = br + (int64_t)(nk - 1) * BK * p.ldb;
      cn = cr;
      sa = 0;
      sb = 0;
    }
    const int64_t ga = NS * BK, gb = (int64_t)NS * BK * p.ldb;   // one group of K steps
    const bool one = ng == 1;
    group(std::true_type{}, one ? an : ar + ga, one ? bn : br + gb, one ? sa : BK,
          one ? sb : (int64_t)BK * p.ldb);
    for (int g = 1; g < ng; ++g) {
      const bool last = g == ng - 1;
      group(std::false_type{}, last ? an : ar + (g + 1) * ga, last ? bn : br + (g + 1) * gb,
            last ? sa : BK, last ? sb : (int64_t)BK * p.ldb);
    }

    // ---- epilogue of tile r: every MFMA of the tile has written its
    // accumulator before they are read (acc_fence keeps the reads after the
    // drain); the next tile's first MFMAs start from srcC = 0, so nothing
    // clears them
    LOOM_WAIT_VMCNT(0);
    mfma_drain();
    acc_fence(acc);
    char* const cb = cr;
    // staging addresses: accumulator tile (tn, tm = 2 qt + h) of this lane
    // goes to row 32 wm + 16 h + lr, chunk (16 wn + 2 tn + lg / 2) ^ lr, i.e.
    // e_lane ^ (tn << 5) + 8 KB h; store row rho = 16 wave + 2 i + lane / 32
    // (tile row 128 (wave / 2) + 32 qt + 16 (wave & 1) + 2 i + lane / 32) is
    // read at r_lane ^ (i << 5) + 1 KB i
    uint32_t e_lane = (uint32_t)((wm * 32 + lr) * 512 + (((wn * 16 + (lg >> 1)) ^ lr) * 16) + (lg & 1) * 8);
    uint32_t r_lane = (uint32_t)((wave * 16 + (lane >> 5)) * 512 + (((lane & 31) ^ (lane >> 5)) * 16));
    asm volatile("" : "+v"(e_lane), "+v"(r_lane));   // computed here, not hoisted and kept live
#pragma unroll
    for (int qt = 0; qt < TT / 2; ++qt) {
#pragma unroll
      for (int tn = 0; tn < TT; ++tn)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tm = 2 * qt + h;
          *(__attribute__((address_space(3))) u32x2_t*)(cst + ((e_lane ^ (uint32_t)(tn << 5)) + h * 8192)) =
              u32x2_t{pack2<H>(acc[tn][tm][0], acc[tn][tm][1]), pack2<H>(acc[tn][tm][2], acc[tn][tm][3])};
        }
      LOOM_WAIT_LGKM0();
      barrier_nofence();
#pragma unroll
      for (int i = 0; i < E_ROWS / 8; ++i) {
        const u32x4_t v =
            *(const __attribute__((address_space(3))) u32x4_t*)(cst + ((r_lane ^ (uint32_t)(i << 5)) + i * 1024));
        char* const sb = cb + (int64_t)(qt * 32 + i * 2) * p.ldc * 2;
        store_stream(reinterpret_cast<u32x4_t*>(sb + st_lane), v);
      }
      LOOM_WAIT_LGKM0();
      barrier_nofence();
    }
    ar = an;
    br = bn;
    cr = cn;
  }
}

// Launches the persistent kernel when every tile is whole, the tiles divide
// evenly over one workgroup per CU (at least two each) and the pipelined
// kernel's conditions hold; the caller falls back otherwise.
template <bool H>
bool launch_persist(const GemmParams& p, bool aligned, bool out_f32, hipStream_t st) {
  const int cus = stream_cus(st);   // 0 when unknown: the persistent kernel is then not used
  const int64_t ntiles = (int64_t)p.tiles_m * p.tiles_n * p.nz;
  const bool ok = aligned && !out_f32 && !p.split && cus >= 8 && cus % 8 == 0 &&
                  p.M % 256 == 0 && p.N % 256 == 0 && p.k_total % 128 == 0 && ntiles % cus == 0 &&
                  ntiles / cus >= 2 && p.lda < (1 << 22) && p.ldb < (1 << 22) && p.ldc < (1 << 22);
  if (!ok) return false;
  hipLaunchKernelGGL((gemm_persist_kernel<H>), dim3((unsigned)cus), dim3(256), 0, st, p,
                     (int)(ntiles / cus));
  return true;
}

// out[e] = bf16( sum_{s ascending} G[s][e] ) -- the split-0 reduction of
// examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:34-51.
template <bool H>
__global__ void __launch_bounds__(256) splitk_reduce_vec4(const float* __restrict__ G,
                                                          uint16_t* __restrict__ out,
                                                          int64_t MN, int S) {
  const int64_t n4 = MN / 4;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n4;
       q += (int64_t)gridDim.x * blockDim.x) {
    f32x4_t s = *reinterpret_cast<const f32x4_t*>(G + q * 4);
    // sixteen slabs' loads in flight at a time (a short last group re-reads
    // slab S-1 in the unused slots), so 17 slabs cost one memory latency;
    // the adds stay in ascending s
    for (int k = 1; k < S; k += 16) {
      f32x4_t v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        v[j] = *reinterpret_cast<const f32x4_t*>(G + (int64_t)min(k + j, S - 1) * MN + q * 4);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (k + j < S) {
          s[0] += v[j][0];
          s[1] += v[j][1];
          s[2] += v[j][2];
          s[3] += v[j][3];
        }
      }
    }
    u32x2_t o{pack2<H>(s[0], s[1]), pack2<H>(s[2], s[3])};
    *reinterpret_cast<u32x2_t*>(out + q * 4) = o;
  }
}

template <bool H>
__global__ void __launch_bounds__(256) splitk_reduce_scalar(const float* __restrict__ G,
                                                            uint16_t* __restrict__ out,
                                                            int64_t MN, int S) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < MN;
       e += (int64_t)gridDim.x * blockDim.x) {
    float s = G[e];
    for (int k = 1; k < S; ++k) s += G[(int64_t)k * MN + e];
    out[e] = (uint16_t)cvt16<H>(s);
  }
}

template <int BM, int BN, int WM, int WN, bool H>
hipError_t launch_tile(const GemmParams& p, bool aligned, bool out_f32, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n * p.nz)), block(64 * WM * WN);
  if (aligned) {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, true, H>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, false, H>), grid, block, 0, st, p);
  } else {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, true, H>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, false, H>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

// Square workgroup tiles built for gfx950; a (tile_m, tile_n) binding runs
// on the smallest one covering both symbols (loom_fit_tile).
constexpr int64_t kGemmTiles[3] = {64, 128, 256};

// Depth of the DMA pipeline of the 256x256 fallback kernel: BK-deep stages,
// NS of them (32 x 4 measured fastest of 32/64 deep, 2-4 stages).
constexpr int kDmaBK = 32, kDmaNS = 4;

template <bool H>
hipError_t launch_gemm(GemmParams p, int64_t tile_m, int64_t tile_n, bool aligned, bool out_f32,
                       hipStream_t st) {
  p.tiles_m = (int)cdiv64(p.M, tile_m);
  p.tiles_n = (int)cdiv64(p.N, tile_n);
  if (tile_m == 64) {
    if (launch_pipe<64, H>(p, aligned, out_f32, st)) return hipGetLastError();
    return launch_tile<64, 64, 1, 2, H>(p, aligned, out_f32, st);
  }
  if (tile_m == 128) {
    if (launch_pipe<128, H>(p, aligned, out_f32, st)) return hipGetLastError();
    return launch_tile<128, 128, 2, 2, H>(p, aligned, out_f32, st);
  }
  if (launch_persist<H>(p, aligned, out_f32, st)) return hipGetLastError();
  if (launch_pipe<256, H>(p, aligned, out_f32, st)) return hipGetLastError();
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n * p.nz)), block(256);
  // otherwise the LDS-DMA kernel needs whole BK steps in every K range
  constexpr int BK = kDmaBK, NS = kDmaNS;
  const bool dma = aligned && p.k_total % BK == 0 && (!p.split || p.k_slab % BK == 0);
  if (dma) {
    if (out_f32)
      hipLaunchKernelGGL((gemm_dma_kernel<BK, NS, true, H>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<BK, NS, false, H>), grid, block, 0, st, p);
    return hipGetLastError();
  }
  return launch_tile<256, 256, 2, 4, H>(p, aligned, out_f32, st);
}

// Checks what every GEMM entry point shares.  On success *wg is the square
// workgroup tile the (tile_m, tile_n) binding runs as: the smallest built tile
// covering both (the largest built one for bindings above it).  Every tile is
// bounded by its loop extent (natural_ub).
int check_gemm_common(const void* a, const void* b, const void* c, int64_t M, int64_t N,
                      int64_t K, int64_t tile_m, int64_t tile_n, int64_t tile_k, int64_t* wg,
                      const char* fn, char* err, size_t errlen) {
  if (!a || !b || !c) return loom_fail(err, errlen, LOOM_EINVAL, "%s: null tensor pointer", fn);
  if (M <= 0 || N <= 0 || K <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: extents must be positive (M=%lld N=%lld K=%lld)",
                     fn, (long long)M, (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: M, N and K must be below 2^30", fn);
  if (tile_m <= 0 || tile_n <= 0 || tile_k <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: tile sizes must be positive", fn);
  const int64_t em = loom_fit_tile(tile_m, M, kGemmTiles, 3);
  const int64_t en = loom_fit_tile(tile_n, N, kGemmTiles, 3);
  if (em == 0 || en == 0 || tile_k > K)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "%s: tiles exceed their extents (natural_ub): tile_m=%lld (M=%lld), "
                     "tile_n=%lld (N=%lld), tile_k=%lld (K=%lld)",
                     fn, (long long)tile_m, (long long)M, (long long)tile_n, (long long)N,
                     (long long)tile_k, (long long)K);
  if (em < 0 || en < 0)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "%s: tile_m=%lld, tile_n=%lld: each must be a multiple of 16 (the MFMA tile "
                     "edge) or its whole extent",
                     fn, (long long)tile_m, (long long)tile_n);
  // square workgroup tiles: the larger of the two covers both symbols
  *wg = std::max(em, en);
  return LOOM_OK;
}

template <bool H>
int matmul_impl(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                    int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                    size_t errlen) {
  int64_t wg = 0;
  int rc = check_gemm_common(x, y, out, M, N, K, tile_m, tile_n, tile_k, &wg, "matmul", err,
                             errlen);
  if (rc) return rc;
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(x);
  p.B = static_cast<const uint16_t*>(y);
  p.C = out;
  p.M = M;
  p.N = N;
  p.lda = K;
  p.ldb = N;
  p.ldc = N;
  p.k_total = K;
  p.k_slab = K;
  p.split = 0;
  p.nz = 1;
  // the vector-store kernels also need a 16-byte-aligned C; others take the
  // register-staged kernel (element stores)
  const bool al = K % 8 == 0 && N % 8 == 0 && aligned16(x) && aligned16(y) && aligned16(out);
  if (loom_validate_only()) return loom_ok(err, errlen);
  (void)launch_gemm<H>(p, wg, wg, al, false, static_cast<hipStream_t>(stream));
  return loom_check_launch(err, errlen, "matmul");
}

template <bool H>
int batch_matmul_impl(const void* arg0, const void* arg1, void* arg2, int64_t Bt, int64_t M,
                          int64_t N, int64_t K, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                          int64_t tile_k, void* stream, char* err, size_t errlen) {
  int64_t wg = 0;
  int rc = check_gemm_common(arg0, arg1, arg2, M, N, K, tile_m, tile_n, tile_k, &wg,
                             "batch_matmul", err, errlen);
  if (rc) return rc;
  if (Bt <= 0 || tile_b <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "batch_matmul: batch and tile_b must be positive");
  if (tile_b > Bt)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "batch_matmul: tile_b=%lld exceeds its extent B=%lld (natural_ub)",
                     (long long)tile_b, (long long)Bt);
  if (!loom_prod_le({cdiv64(M, wg), cdiv64(N, wg), Bt}, 0x7fffffff) ||
      !loom_prod_le({Bt, M, K}, (int64_t)1 << 50) || !loom_prod_le({Bt, N, K}, (int64_t)1 << 50) ||
      !loom_prod_le({Bt, M, N}, (int64_t)1 << 50))
    return loom_fail(err, errlen, LOOM_EINVAL, "batch_matmul: problem too large");
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(arg0);
  p.B = static_cast<const uint16_t*>(arg1);
  p.C = arg2;
  p.M = M;
  p.N = N;
  p.lda = K;
  p.ldb = N;
  p.ldc = N;
  p.za = M * K;
  p.zb = K * N;
  p.zc = M * N;
  p.k_total = K;
  p.k_slab = K;
  p.split = 0;
  p.nz = (int)Bt;
  const bool al =
      K % 8 == 0 && N % 8 == 0 && aligned16(arg0) && aligned16(arg1) && aligned16(arg2);
  if (loom_validate_only()) return loom_ok(err, errlen);
  (void)launch_gemm<H>(p, wg, wg, al, false, static_cast<hipStream_t>(stream));
  return loom_check_launch(err, errlen, "batch_matmul");
}


template <bool H>
int split_k_matmul_gather_impl(const void* a, const void* b, void* out, void* partials,
                                   size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                   int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
                                   char* err, size_t errlen) {
  int64_t wg = 0;
  int rc = check_gemm_common(a, b, out, M, N, K, tile_m, tile_n, tile_k, &wg,
                             "split_k_matmul_gather", err, errlen);
  if (rc) return rc;
  const int64_t S = cdiv64(K, tile_k);
  if (!loom_prod_le({S, cdiv64(M, wg), cdiv64(N, wg)}, 0x7fffffff) ||
      !loom_prod_le({S, M, N}, (int64_t)1 << 46) || !loom_prod_le({M, K}, (int64_t)1 << 50) ||
      !loom_prod_le({N, K}, (int64_t)1 << 50))
    return loom_fail(err, errlen, LOOM_EINVAL, "split_k_matmul_gather: problem too large");
  const size_t need = loom_hip_split_k_workspace_bytes(M, N, K, tile_k);
  if (!partials || partials_bytes < need)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "split_k_matmul_gather: partials workspace needs %zu bytes, got %zu", need,
                     partials_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(a);
  p.B = static_cast<const uint16_t*>(b);
  p.C = partials;
  p.M = M;
  p.N = N;
  p.lda = K;
  p.ldb = N;
  p.ldc = N;
  p.zc = M * N;
  p.k_total = K;
  p.k_slab = tile_k;
  p.split = 1;
  p.nz = (int)S;
  const bool al = K % 8 == 0 && N % 8 == 0 && tile_k % 8 == 0 && aligned16(a) && aligned16(b) &&
                  aligned16(partials);
  if (loom_validate_only()) return loom_ok(err, errlen);
  (void)launch_gemm<H>(p, wg, wg, al, true, st);
  rc = loom_check_launch(err, errlen, "split_k_matmul_gather (slab GEMM)");
  if (rc) return rc;
  const int64_t MN = M * N;
  if (MN % 4 == 0 && aligned16(partials) && (reinterpret_cast<uintptr_t>(out) & 7u) == 0) {
    const int64_t blocks = std::min<int64_t>(cdiv64(MN / 4, 256), 8192);
    hipLaunchKernelGGL(splitk_reduce_vec4<H>, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const float*>(partials), static_cast<uint16_t*>(out), MN,
                       (int)S);
  } else {
    const int64_t blocks = std::min<int64_t>(cdiv64(MN, 256), 8192);
    hipLaunchKernelGGL(splitk_reduce_scalar<H>, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const float*>(partials), static_cast<uint16_t*>(out), MN,
                       (int)S);
  }
  return loom_check_launch(err, errlen, "split_k_matmul_gather (gather-reduce)");
}

}  // namespace

extern "C" {

size_t loom_hip_split_k_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t tile_k) {
  if (M <= 0 || N <= 0 || K <= 0 || tile_k <= 0) return 0;
  // a product that does not fit is reported as no size at all fits
  if (!loom_prod_le({cdiv64(K, tile_k), M, N, 4}, INT64_MAX)) return SIZE_MAX;
  return (size_t)cdiv64(K, tile_k) * (size_t)M * (size_t)N * sizeof(float);
}

int loom_hip_matmul(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                    int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                    size_t errlen) {
  return matmul_impl<false>(x, y, out, M, N, K, tile_m, tile_n, tile_k, stream, err, errlen);
}
int loom_hip_matmul_f16(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                        int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                        size_t errlen) {
  return matmul_impl<true>(x, y, out, M, N, K, tile_m, tile_n, tile_k, stream, err, errlen);
}
int loom_hip_batch_matmul(const void* arg0, const void* arg1, void* arg2, int64_t B, int64_t M,
                          int64_t N, int64_t K, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                          int64_t tile_k, void* stream, char* err, size_t errlen) {
  return batch_matmul_impl<false>(arg0, arg1, arg2, B, M, N, K, tile_b, tile_m, tile_n, tile_k,
                                  stream, err, errlen);
}
int loom_hip_batch_matmul_f16(const void* arg0, const void* arg1, void* arg2, int64_t B,
                              int64_t M, int64_t N, int64_t K, int64_t tile_b, int64_t tile_m,
                              int64_t tile_n, int64_t tile_k, void* stream, char* err,
                              size_t errlen) {
  return batch_matmul_impl<true>(arg0, arg1, arg2, B, M, N, K, tile_b, tile_m, tile_n, tile_k,
                                 stream, err, errlen);
}
int loom_hip_split_k_matmul_gather(const void* a, const void* b, void* out, void* partials,
                                   size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                   int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
                                   char* err, size_t errlen) {
  return split_k_matmul_gather_impl<false>(a, b, out, partials, partials_bytes, M, N, K, tile_m,
                                           tile_n, tile_k, stream, err, errlen);
}
int loom_hip_split_k_matmul_gather_f16(const void* a, const void* b, void* out, void* partials,
                                       size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                       int64_t tile_m, int64_t tile_n, int64_t tile_k,
                                       void* stream, char* err, size_t errlen) {
  return split_k_matmul_gather_impl<true>(a, b, out, partials, partials_bytes, M, N, K, tile_m,
                                          tile_n, tile_k, stream, err, errlen);
}

}  // extern "C"
