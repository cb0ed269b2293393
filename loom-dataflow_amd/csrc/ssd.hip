// ssd.hip -- Mamba-2 SSD prologue on gfx950: the kernels that turn raw
// (x, dt, A, B, C) into the inputs of @helion_mamba2_chunk_scan_kernel
// (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4 takes cb,
// dA_cumsum and prev_states_T ready-made; the reference repository has no
// code that produces them).  The three stages follow the published SSD
// algorithm (Dao & Gu 2024, "Transformers are SSMs"), chunked form:
//
//   dA_cumsum[b,h,c,q] = sum_{q' <= q} dt[b,h,cQ+q'] * A[h]
//   cb[b,c,g,i,j]      = sum_n C[b,g,cQ+i,n] B[b,g,cQ+j,n]   (j <= i, else 0)
//   states[b,c,h,n,p]  = sum_k B[b,g,cQ+k,n] w_c[k] x[b,h,cQ+k,p],
//                        w_c[k] = exp(dA[c,Q-1] - dA[c,k]) dt[c,k]
//   prev_states_T[b,0] = 0,
//   prev_states_T[b,c] = exp(dA[c-1,Q-1]) prev_states_T[b,c-1] + states[b,c-1]
//
// with g = h / (H / G).  dt [b,H,L] already has the layout of [b,H,c,Q],
// so chunk_scan reads the caller's dt unchanged.
//
// gfx950 mapping:
//   ssd_cumsum_kernel  one wave per (b,h,c): per-lane serial sums, then a
//                      wave prefix scan of the lane totals (DPP shuffles).
//   ssd_cb_kernel      one wave per (b,c,g, 16-row band): MFMA D = B . C^T
//                      over n, straight from global memory (both operands
//                      are n-contiguous rows); the transposed tile gives each
//                      lane four consecutive j of one row i (8-byte stores).
//   ssd_state_kernel   one workgroup per (b, h, 64-wide n block) walks the
//                      chunks in order, keeping prev_states in the MFMA
//                      accumulators: per chunk it stores prev(c), scales by
//                      exp(dA[c,Q-1]) and accumulates states(c), so the
//                      chunk states never reach HBM.  x and B chunks are
//                      staged in LDS ([k][p], [k][n]) and read as MFMA
//                      operands with ds_read_b64_tr_b16; w_c scales B in
//                      fp32 and enters the MFMA as a bf16 hi + lo pair.
#include "common.h"

namespace {

// ---------------------------------------------------------------------------
// dA_cumsum
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) ssd_cumsum_kernel(const float* __restrict__ dt,
                                                        const float* __restrict__ A,
                                                        float* __restrict__ dA, int H, int nc,
                                                        int Q, int per_lane) {
  const int row = blockIdx.x;                  // (b*H + h)*nc + c
  const int lane = threadIdx.x;
  const int h = (row / nc) % H;
  const float a = A[h];
  const float* src = dt + (int64_t)row * Q;
  float* dst = dA + (int64_t)row * Q;
  const int q0 = lane * per_lane;
  float v[8];
  float run = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int q = q0 + e;
    const float d = (e < per_lane && q < Q) ? src[q] : 0.f;
    run += __fmul_rn(d, a);
    v[e] = run;
  }
  // exclusive prefix of the lane totals
  float incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  const float base = incl - run;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int q = q0 + e;
    if (e < per_lane && q < Q) dst[q] = base + v[e];
  }
}

// ---------------------------------------------------------------------------
// cb = C B^T, lower triangle
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) ssd_cb_kernel(const uint16_t* __restrict__ Bm,
                                                    const uint16_t* __restrict__ Cm,
                                                    uint16_t* __restrict__ cb, int nc, int G,
                                                    int L, int Q, int N) {
  const int bcg = blockIdx.x;                  // (b*nc + c)*G + g
  const int it = blockIdx.y;                   // 16-row band of i
  const int lane = threadIdx.x, r = lane & 15, gq = lane >> 4;
  const int g = bcg % G, c = (bcg / G) % nc, b = bcg / (G * nc);
  const int64_t rowbase = ((int64_t)(b * G + g) * L + (int64_t)c * Q);
  const uint16_t* Cc = Cm + rowbase * N;
  const uint16_t* Bc = Bm + rowbase * N;
  uint16_t* out = cb + (int64_t)bcg * Q * Q;
  const int i0 = 16 * it;
  const int nks = (N + 31) / 32;
  // C^T operand: lane holds C[i0 + r][32 ks + 8 gq .. + 7] (zero past N)
  u32x4_t cf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int n = 32 * ks + 8 * gq;
    cf[ks] = (ks < nks && n < N) ? *reinterpret_cast<const u32x4_t*>(Cc + (int64_t)(i0 + r) * N + n)
                                 : u32x4_t{0u, 0u, 0u, 0u};
  }
  for (int jt = 0; jt < Q / 16; ++jt) {
    uint16_t* orow = out + (int64_t)(i0 + r) * Q + 16 * jt + 4 * gq;
    if (jt > it) {
      *reinterpret_cast<u32x2_t*>(orow) = u32x2_t{0u, 0u};
      continue;
    }
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < nks) {
        const int n = 32 * ks + 8 * gq;
        const u32x4_t bf = n < N ? *reinterpret_cast<const u32x4_t*>(Bc + (int64_t)(16 * jt + r) * N + n)
                                 : u32x4_t{0u, 0u, 0u, 0u};
        acc = mfma16(bf, cf[ks], acc);        // D[j][i] = sum_n B[j][n] C[i][n]
      }
    }
    // lane holds cb[i0 + r][16 jt + 4 gq + e]
    if (jt == it) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * gq + e > r) acc[e] = 0.f;
    }
    *reinterpret_cast<u32x2_t*>(orow) =
        u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
  }
}

// ---------------------------------------------------------------------------
// chunk states + state passing -> prev_states_T
// ---------------------------------------------------------------------------
constexpr int kSsdQmax = 256, kSsdPmax = 256, kSsdNB = 64, kSsdWaves = 8;
constexpr int kSsdXBytes = 64 * 1024;        // x chunk [Qpad][P] bf16 at most

template <int TPW>
__global__ void __launch_bounds__(64 * kSsdWaves) ssd_state_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ dt, const float* __restrict__ dA,
    const uint16_t* __restrict__ Bm, float* __restrict__ prevT, int H, int G, int nc, int Q,
    int P, int N, int nb) {
  // LDS: x chunk [Qpad][P], B chunk [Qpad][nb] (bf16), w [Qpad]
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kSsdXBytes / 2];
  __shared__ __attribute__((aligned(16))) uint16_t s_b[kSsdQmax * kSsdNB];
  __shared__ __attribute__((aligned(16))) float s_w[kSsdQmax];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, gq = lane >> 4, a4 = r >> 2, c4 = r & 3;
  const int bh = blockIdx.x, nblk = blockIdx.y;
  const int b = bh / H, h = bh % H, g = h / (H / G);
  const int n0 = nblk * nb;
  const int L = nc * Q, Qpad = (Q + 31) & ~31;
  const int XR = P * 2, BR = nb * 2;           // LDS row bytes
  const int ptiles = P / 16, ntiles = nb / 16, tiles = ptiles * ntiles;

  const uint16_t* xg = x + ((int64_t)bh * L) * P;
  const uint16_t* bg = Bm + ((int64_t)(b * G + g) * L) * N + n0;
  const float* dAg = dA + (int64_t)bh * nc * Q;
  const float* dtg = dt + (int64_t)bh * nc * Q;

  // staging: x rows (P*2 bytes) and B rows (nb*2 bytes) of chunk c, 16 bytes a piece
  const int xpieces = Qpad * P / 8, bpieces = Qpad * nb / 8;
  constexpr int kMaxPieces = (kSsdXBytes / 16 + kSsdQmax * kSsdNB / 8) / (64 * kSsdWaves);
  u32x4_t pre[kMaxPieces];
  float wpre = 0.f;
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int u = 0; u < kMaxPieces; ++u) {
      const int idx = tid + u * 64 * kSsdWaves;
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (idx < xpieces) {
        const int k = idx / (P / 8), pc = idx % (P / 8);
        if (k < Q) v = *reinterpret_cast<const u32x4_t*>(xg + ((int64_t)c * Q + k) * P + pc * 8);
      } else if (idx < xpieces + bpieces) {
        const int j = idx - xpieces;
        const int k = j / (nb / 8), nc8 = j % (nb / 8);
        if (k < Q) v = *reinterpret_cast<const u32x4_t*>(bg + ((int64_t)c * Q + k) * N + nc8 * 8);
      }
      pre[u] = v;
    }
    wpre = 0.f;
    if (tid < Q) {
      const float last = dAg[(int64_t)c * Q + Q - 1];
      wpre = expf(last - dAg[(int64_t)c * Q + tid]) * dtg[(int64_t)c * Q + tid];
    }
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int u = 0; u < kMaxPieces; ++u) {
      const int idx = tid + u * 64 * kSsdWaves;
      if (idx < xpieces)
        *reinterpret_cast<u32x4_t*>(&s_x[idx * 8]) = pre[u];
      else if (idx < xpieces + bpieces)
        *reinterpret_cast<u32x4_t*>(&s_b[(idx - xpieces) * 8]) = pre[u];
    }
    if (tid < Qpad) s_w[tid] = wpre;
  };

  // running prev_states^T tiles: tile t = wave + 8 u -> (pt, nt); lane holds
  // prev[n0 + 16 nt + r][16 pt + 4 gq + e]
  f32x4_t R[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) R[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_chunk(0);
  store_chunk();
  __syncthreads();
  for (int c = 0; c < nc; ++c) {
    if (c + 1 < nc) load_chunk(c + 1);         // in flight during this chunk's MFMAs
    // prev(c), then R = exp(dA[c, Q-1]) R + states(c)
    const float decay = expf(dAg[(int64_t)c * Q + Q - 1]);
    float* outc = prevT + (((int64_t)(b * nc + c) * H + h) * N + n0) * P;
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int t = wave + kSsdWaves * u;
      if (t < tiles) {
        const int pt = t % ptiles, nt = t / ptiles;
        *reinterpret_cast<f32x4_t*>(outc + (int64_t)(16 * nt + r) * P + 16 * pt + 4 * gq) = R[u];
        R[u] *= decay;
      }
    }
    const char* xs = reinterpret_cast<const char*>(s_x);
    const char* bs = reinterpret_cast<const char*>(s_b);
    for (int ks = 0; ks < Qpad / 32; ++ks) {
      const int k0 = 32 * ks + 4 * gq;          // rows k0 + a4 (lo) and + 16 (hi)
      const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(&s_w[k0]);
      const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(&s_w[k0 + 16]);
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        const int t = wave + kSsdWaves * u;
        if (t < tiles) {
          const int pt = t % ptiles, nt = t / ptiles;
          // x^T operand: p = 16 pt + r, k in {k0..k0+3, k0+16..k0+19}
          const lds_char_t* qx = (const lds_char_t*)(xs + (k0 + a4) * XR + (2 * pt + (c4 >> 1)) * 16 + (c4 & 1) * 8);
          const u32x2_t xlo = lds_read_tr16(qx), xhi = lds_read_tr16(qx + 16 * XR);
          const u32x4_t xf = u32x4_t{xlo[0], xlo[1], xhi[0], xhi[1]};
          // (w B) operand: n = 16 nt + r, same k
          const lds_char_t* qb = (const lds_char_t*)(bs + (k0 + a4) * BR + (2 * nt + (c4 >> 1)) * 16 + (c4 & 1) * 8);
          const u32x2_t blo = lds_read_tr16(qb), bhi = lds_read_tr16(qb + 16 * BR);
          const float v[8] = {bf2f_lo(blo[0]) * w0[0], bf2f_hi(blo[0]) * w0[1],
                              bf2f_lo(blo[1]) * w0[2], bf2f_hi(blo[1]) * w0[3],
                              bf2f_lo(bhi[0]) * w1[0], bf2f_hi(bhi[0]) * w1[1],
                              bf2f_lo(bhi[1]) * w1[2], bf2f_hi(bhi[1]) * w1[3]};
          u32x4_t hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hi[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
            lo[e] = pack_bf16x2(v[2 * e] - bf2f_lo(hi[e]), v[2 * e + 1] - bf2f_hi(hi[e]));
          }
          R[u] = mfma16(xf, hi, R[u]);
          R[u] = mfma16(xf, lo, R[u]);
        }
      }
    }
    __syncthreads();
    if (c + 1 < nc) {
      store_chunk();
      __syncthreads();
    }
  }
}

template <int TPW>
void launch_state(const uint16_t* x, const float* dt, const float* dA, const uint16_t* Bm,
                  float* prevT, int Bb, int H, int G, int nc, int Q, int P, int N, int nb,
                  hipStream_t st) {
  hipLaunchKernelGGL((ssd_state_kernel<TPW>), dim3((unsigned)(Bb * H), (unsigned)(N / nb)),
                     dim3(64 * kSsdWaves), 0, st, x, dt, dA, Bm, prevT, H, G, nc, Q, P, N, nb);
}

int check_ssd(const char* fn, int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
              int64_t chunk_size, int64_t headdim, int64_t dstate, char* err, size_t errlen) {
  if (batch <= 0 || nchunks <= 0 || nheads <= 0 || ngroups <= 0 || chunk_size <= 0 ||
      headdim <= 0 || dstate <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: extents must be positive", fn);
  if (nheads % ngroups != 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: nheads %lld not a multiple of ngroups %lld",
                     fn, (long long)nheads, (long long)ngroups);
  if (chunk_size % 16 || headdim % 16 || dstate % 16)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: chunk_size, headdim and dstate must be multiples of 16", fn);
  if (chunk_size > kSsdQmax || headdim > kSsdPmax || dstate > 128 || (dstate > 32 && dstate % 32))
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: built for chunk_size <= %d, headdim <= %d, dstate <= 128 "
                     "(a multiple of 32 above 32)",
                     fn, kSsdQmax, kSsdPmax);
  if (((chunk_size + 31) & ~31) * headdim * 2 > kSsdXBytes)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: chunk_size x headdim above the %d-byte LDS chunk buffer", fn, kSsdXBytes);
  if (batch * nheads * nchunks * chunk_size * headdim >= (int64_t)1 << 40)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: problem too large", fn);
  return LOOM_OK;
}

}  // namespace

extern "C" {

int loom_hip_ssd_chunk_cumsum(const void* dt, const void* A, void* dA_cumsum, int64_t batch,
                              int64_t nchunks, int64_t nheads, int64_t chunk_size, void* stream,
                              char* err, size_t errlen) {
  if (!dt || !A || !dA_cumsum)
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_cumsum: null tensor pointer");
  if (batch <= 0 || nchunks <= 0 || nheads <= 0 || chunk_size <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_cumsum: extents must be positive");
  if (chunk_size > 512)
    return loom_fail(err, errlen, LOOM_EUNSUP, "ssd_chunk_cumsum: chunk_size above 512");
  if (batch * nheads * nchunks > 0x7fffffff / 64)
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_cumsum: problem too large");
  const int per_lane = (int)((chunk_size + 63) / 64);
  hipLaunchKernelGGL(ssd_cumsum_kernel, dim3((unsigned)(batch * nheads * nchunks)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(dt),
                     static_cast<const float*>(A), static_cast<float*>(dA_cumsum), (int)nheads,
                     (int)nchunks, (int)chunk_size, per_lane);
  return loom_check_launch(err, errlen, "ssd_chunk_cumsum");
}

int loom_hip_ssd_bmm_chunk(const void* B, const void* C, void* cb, int64_t batch, int64_t nchunks,
                           int64_t ngroups, int64_t chunk_size, int64_t dstate, void* stream,
                           char* err, size_t errlen) {
  if (!B || !C || !cb) return loom_fail(err, errlen, LOOM_EINVAL, "ssd_bmm_chunk: null tensor pointer");
  int rc = check_ssd("ssd_bmm_chunk", batch, nchunks, ngroups, ngroups, chunk_size, 16, dstate,
                     err, errlen);
  if (rc) return rc;
  if (!aligned16(B) || !aligned16(C) || (reinterpret_cast<uintptr_t>(cb) & 7u))
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_bmm_chunk: B, C 16-byte and cb 8-byte aligned");
  hipLaunchKernelGGL(ssd_cb_kernel, dim3((unsigned)(batch * nchunks * ngroups), (unsigned)(chunk_size / 16)),
                     dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(B), static_cast<const uint16_t*>(C),
                     static_cast<uint16_t*>(cb), (int)nchunks, (int)ngroups,
                     (int)(nchunks * chunk_size), (int)chunk_size, (int)dstate);
  return loom_check_launch(err, errlen, "ssd_bmm_chunk");
}

int loom_hip_ssd_chunk_state_passing(const void* x, const void* dt, const void* dA_cumsum,
                                     const void* B, void* prev_states_T, int64_t batch,
                                     int64_t nchunks, int64_t nheads, int64_t ngroups,
                                     int64_t chunk_size, int64_t headdim, int64_t dstate,
                                     void* stream, char* err, size_t errlen) {
  if (!x || !dt || !dA_cumsum || !B || !prev_states_T)
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_state_passing: null tensor pointer");
  int rc = check_ssd("ssd_chunk_state_passing", batch, nchunks, nheads, ngroups, chunk_size,
                     headdim, dstate, err, errlen);
  if (rc) return rc;
  if (!aligned16(x) || !aligned16(B) || !aligned16(prev_states_T))
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_state_passing: tensors must be 16-byte aligned");
  // n block: 64 wide while the P x 64 block fits four tiles per wave, else 32
  const int nb = (int)std::min<int64_t>(dstate, headdim <= 128 ? kSsdNB : 32);
  const int tiles = (int)(headdim / 16) * (nb / 16);
  const int tpw = (tiles + kSsdWaves - 1) / kSsdWaves;
  if (dstate % nb != 0 || tpw > 4)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "ssd_chunk_state_passing: dstate %lld with headdim %lld not built",
                     (long long)dstate, (long long)headdim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* dtp = static_cast<const float*>(dt);
  const auto* dAp = static_cast<const float*>(dA_cumsum);
  const auto* bp = static_cast<const uint16_t*>(B);
  auto* pp = static_cast<float*>(prev_states_T);
  const int Bb = (int)batch, H = (int)nheads, G = (int)ngroups, nc = (int)nchunks,
            Q = (int)chunk_size, P = (int)headdim, N = (int)dstate;
  if (tpw <= 1) launch_state<1>(xp, dtp, dAp, bp, pp, Bb, H, G, nc, Q, P, N, nb, st);
  else if (tpw <= 2) launch_state<2>(xp, dtp, dAp, bp, pp, Bb, H, G, nc, Q, P, N, nb, st);
  else launch_state<4>(xp, dtp, dAp, bp, pp, Bb, H, G, nc, Q, P, N, nb, st);
  return loom_check_launch(err, errlen, "ssd_chunk_state_passing");
}

int loom_hip_ssd_prologue(const void* x, const void* dt, const void* A, const void* B,
                          const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                          int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                          int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                          char* err, size_t errlen) {
  int rc = check_ssd("ssd_prologue", batch, nchunks, nheads, ngroups, chunk_size, headdim, dstate,
                     err, errlen);
  if (rc) return rc;
  rc = loom_hip_ssd_chunk_cumsum(dt, A, dA_cumsum, batch, nchunks, nheads, chunk_size, stream,
                                 err, errlen);
  if (rc) return rc;
  rc = loom_hip_ssd_bmm_chunk(B, C, cb, batch, nchunks, ngroups, chunk_size, dstate, stream, err,
                              errlen);
  if (rc) return rc;
  return loom_hip_ssd_chunk_state_passing(x, dt, dA_cumsum, B, prev_states_T, batch, nchunks,
                                          nheads, ngroups, chunk_size, headdim, dstate, stream,
                                          err, errlen);
}

}  // extern "C"
