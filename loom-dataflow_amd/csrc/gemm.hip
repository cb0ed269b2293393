// gemm.hip -- bf16 GEMM family on gfx950 MFMA: @matmul, @batch_matmul and
// @split_k_matmul_gather (the K-slab GEMM plus its fp32 gather-reduce).
//
// Reference semantics (all three accumulate sum_k x[i,k] * y[k,j]):
//   @matmul                 examples/mm/IR/00_from_helion_frontend.mlir:2-35
//   @batch_matmul           examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4-44
//   @split_k_matmul_gather  examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2-56
// Operands are row-major: A [M,K], B [K,N], C [M,N] (per batch for bmm).
//
// Kernel shape: one workgroup per (tile_m x tile_n) output tile, the grid
// flattened over (z, tile) with z = batch (bmm) or K-slab (split-K).  The
// K loop stages 64-deep A and B tiles through LDS, double buffered, one
// barrier per step:
//   - half of the threads copy A rows (16-byte chunks, coalesced);
//   - the other half copy B as 8x8 blocks (eight 16-byte row loads), transpose
//     each block in registers and store B^T, so both MFMA operands are read
//     as one 16-byte LDS load per lane (k contiguous);
//   - LDS rows are 128 bytes with the 16-byte chunk index XOR-swizzled by
//     (row & 7), which keeps the MFMA operand reads and the transposed B
//     stores free of bank conflicts without padding.
// Each wave owns a (tile_m/WM) x (tile_n/WN) sub-tile of 16x16 fp32
// accumulators fed by v_mfma_f32_16x16x32_bf16.
#include "common.h"

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

template <int BM, int BN, int WM, int WN, bool ALIGNED, bool OUT_F32>
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
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
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
            static_cast<uint16_t*>(p.C)[coff + row * p.ldc + col] = (uint16_t)f2bf(acc[i][j][r]);
        }
      }
    }
  }
}

// out[e] = bf16( sum_{s ascending} G[s][e] ) -- the split-0 reduction of
// examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:34-51.
__global__ void __launch_bounds__(256) splitk_reduce_vec4(const float* __restrict__ G,
                                                          uint16_t* __restrict__ out,
                                                          int64_t MN, int S) {
  const int64_t n4 = MN / 4;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n4;
       q += (int64_t)gridDim.x * blockDim.x) {
    f32x4_t s = *reinterpret_cast<const f32x4_t*>(G + q * 4);
    for (int k = 1; k < S; ++k) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(G + (int64_t)k * MN + q * 4);
      s[0] += v[0];
      s[1] += v[1];
      s[2] += v[2];
      s[3] += v[3];
    }
    u32x2_t o{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
    *reinterpret_cast<u32x2_t*>(out + q * 4) = o;
  }
}

__global__ void __launch_bounds__(256) splitk_reduce_scalar(const float* __restrict__ G,
                                                            uint16_t* __restrict__ out,
                                                            int64_t MN, int S) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < MN;
       e += (int64_t)gridDim.x * blockDim.x) {
    float s = G[e];
    for (int k = 1; k < S; ++k) s += G[(int64_t)k * MN + e];
    out[e] = (uint16_t)f2bf(s);
  }
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_tile(const GemmParams& p, bool aligned, bool out_f32, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n * p.nz)), block(64 * WM * WN);
  if (aligned) {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, true>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, false>), grid, block, 0, st, p);
  } else {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, true>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, false>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

// Workgroup tiles built for gfx950: (tile_m, tile_n) -> waves (WM x WN).
bool tile_supported(int64_t tm, int64_t tn) {
  return (tm == 64 && tn == 64) || (tm == 128 && tn == 128) || (tm == 256 && tn == 256);
}

hipError_t launch_gemm(GemmParams p, int64_t tile_m, int64_t tile_n, bool aligned, bool out_f32,
                       hipStream_t st) {
  p.tiles_m = (int)cdiv64(p.M, tile_m);
  p.tiles_n = (int)cdiv64(p.N, tile_n);
  if (tile_m == 64) return launch_tile<64, 64, 1, 2>(p, aligned, out_f32, st);
  if (tile_m == 128) return launch_tile<128, 128, 2, 2>(p, aligned, out_f32, st);
  return launch_tile<256, 256, 2, 4>(p, aligned, out_f32, st);
}

int check_gemm_common(const void* a, const void* b, const void* c, int64_t M, int64_t N,
                      int64_t K, int64_t tile_m, int64_t tile_n, int64_t tile_k, const char* fn,
                      char* err, size_t errlen) {
  if (!a || !b || !c) return loom_fail(err, errlen, LOOM_EINVAL, "%s: null tensor pointer", fn);
  if (M <= 0 || N <= 0 || K <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: extents must be positive (M=%lld N=%lld K=%lld)",
                     fn, (long long)M, (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30))
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: M and N must be below 2^30", fn);
  if (tile_m <= 0 || tile_n <= 0 || tile_k <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: tile sizes must be positive", fn);
  if (!tile_supported(tile_m, tile_n))
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: workgroup tile %lldx%lld not built for gfx950 (built: 64x64, 128x128, "
                     "256x256)",
                     fn, (long long)tile_m, (long long)tile_n);
  return LOOM_OK;
}

}  // namespace

extern "C" {

int loom_hip_matmul(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                    int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                    size_t errlen) {
  int rc = check_gemm_common(x, y, out, M, N, K, tile_m, tile_n, tile_k, "matmul", err, errlen);
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
  const bool al = K % 8 == 0 && N % 8 == 0 && aligned16(x) && aligned16(y);
  (void)launch_gemm(p, tile_m, tile_n, al, false, static_cast<hipStream_t>(stream));
  return loom_check_launch(err, errlen, "matmul");
}

int loom_hip_batch_matmul(const void* arg0, const void* arg1, void* arg2, int64_t Bt, int64_t M,
                          int64_t N, int64_t K, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                          int64_t tile_k, void* stream, char* err, size_t errlen) {
  int rc = check_gemm_common(arg0, arg1, arg2, M, N, K, tile_m, tile_n, tile_k, "batch_matmul",
                             err, errlen);
  if (rc) return rc;
  if (Bt <= 0 || tile_b <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "batch_matmul: batch and tile_b must be positive");
  const int64_t tiles = cdiv64(M, tile_m) * cdiv64(N, tile_n) * Bt;
  if (tiles > 0x7fffffff)
    return loom_fail(err, errlen, LOOM_EINVAL, "batch_matmul: grid too large");
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
  const bool al = K % 8 == 0 && N % 8 == 0 && aligned16(arg0) && aligned16(arg1);
  (void)launch_gemm(p, tile_m, tile_n, al, false, static_cast<hipStream_t>(stream));
  return loom_check_launch(err, errlen, "batch_matmul");
}

size_t loom_hip_split_k_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t tile_k) {
  if (M <= 0 || N <= 0 || K <= 0 || tile_k <= 0) return 0;
  return (size_t)cdiv64(K, tile_k) * (size_t)M * (size_t)N * sizeof(float);
}

int loom_hip_split_k_matmul_gather(const void* a, const void* b, void* out, void* partials,
                                   size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                   int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
                                   char* err, size_t errlen) {
  int rc = check_gemm_common(a, b, out, M, N, K, tile_m, tile_n, tile_k, "split_k_matmul_gather",
                             err, errlen);
  if (rc) return rc;
  if (tile_k > K)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "split_k_matmul_gather: tile_k=%lld exceeds K=%lld", (long long)tile_k,
                     (long long)K);
  const int64_t S = cdiv64(K, tile_k);
  const size_t need = loom_hip_split_k_workspace_bytes(M, N, K, tile_k);
  if (!partials || partials_bytes < need)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "split_k_matmul_gather: partials workspace needs %zu bytes, got %zu", need,
                     partials_bytes);
  if (S * cdiv64(M, tile_m) * cdiv64(N, tile_n) > 0x7fffffff)
    return loom_fail(err, errlen, LOOM_EINVAL, "split_k_matmul_gather: grid too large");
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
  const bool al = K % 8 == 0 && N % 8 == 0 && tile_k % 8 == 0 && aligned16(a) && aligned16(b);
  (void)launch_gemm(p, tile_m, tile_n, al, true, st);
  rc = loom_check_launch(err, errlen, "split_k_matmul_gather (slab GEMM)");
  if (rc) return rc;
  const int64_t MN = M * N;
  if (MN % 4 == 0 && aligned16(partials) && (reinterpret_cast<uintptr_t>(out) & 7u) == 0) {
    const int64_t blocks = std::min<int64_t>(cdiv64(MN / 4, 256), 8192);
    hipLaunchKernelGGL(splitk_reduce_vec4, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const float*>(partials), static_cast<uint16_t*>(out), MN,
                       (int)S);
  } else {
    const int64_t blocks = std::min<int64_t>(cdiv64(MN, 256), 8192);
    hipLaunchKernelGGL(splitk_reduce_scalar, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const float*>(partials), static_cast<uint16_t*>(out), MN,
                       (int)S);
  }
  return loom_check_launch(err, errlen, "split_k_matmul_gather (gather-reduce)");
}

}  // extern "C"
