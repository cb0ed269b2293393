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
//   ssd_cb_kernel      one wave per (b,c,g, 16-row band, four 16-column
//                      tiles): MFMA D = B . C^T over n, straight from global
//                      memory (both operands are n-contiguous rows), every
//                      load issued before the first MFMA; the transposed
//                      tile gives each lane four consecutive j of one row i
//                      (8-byte stores).
//   ssd_state_kernel   one workgroup per (b, h, 64-wide n block) walks the
//                      chunks in order, keeping prev_states in the MFMA
//                      accumulators: per chunk it stores prev(c), scales by
//                      exp(dA[c,Q-1]) and accumulates states(c), so the
//                      chunk states never reach HBM.  x and B chunks are
//                      staged in LDS ([k][p], [k][n]) and read as MFMA
//                      operands with ds_read_b64_tr_b16; w_c scales x in
//                      fp32 and enters the MFMA as a bf16 hi + lo pair.
#include "common.h"

namespace {

// ---------------------------------------------------------------------------
// dA_cumsum
// ---------------------------------------------------------------------------
// one wave per (b, h, c) row
LOOM_DEV void cumsum_row(const float* __restrict__ dt, const float* __restrict__ A,
                         float* __restrict__ dA, int H, int nc, int Q, int per_lane,
                         int row /* (b*H + h)*nc + c */, int lane) {
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

__global__ void __launch_bounds__(64) ssd_cumsum_kernel(const float* __restrict__ dt,
                                                        const float* __restrict__ A,
                                                        float* __restrict__ dA, int H, int nc,
                                                        int Q, int per_lane) {
  cumsum_row(dt, A, dA, H, nc, Q, per_lane, blockIdx.x, threadIdx.x);
}

// ---------------------------------------------------------------------------
// cb = C B^T, lower triangle
// ---------------------------------------------------------------------------
constexpr int kCbTiles = 4;  // 16x16 output tiles per wave (one row band)
// NKS: 32-wide n steps held in registers (4: dstate <= 128, 8: <= 256)
// one wave per (b, c, g) chunk bcg = (b*nc + c)*G + g, 16-row band `it` of
// i and kCbTiles 16-column tiles of j from jz kCbTiles on
template <bool F16, int NKS>
LOOM_DEV void cb_tiles(const uint16_t* __restrict__ Bm, const uint16_t* __restrict__ Cm,
                       uint16_t* __restrict__ cb, int nc, int G, int L, int Q, int N, int bcg,
                       int it, int jz, int lane) {
  const int jt0 = kCbTiles * jz;               // first 16-column tile of j
  const int r = lane & 15, gq = lane >> 4;
  const int g = bcg % G, c = (bcg / G) % nc, b = bcg / (G * nc);
  const int64_t rowbase = ((int64_t)(b * G + g) * L + (int64_t)c * Q);
  const uint16_t* Cc = Cm + rowbase * N;
  const uint16_t* Bc = Bm + rowbase * N;
  uint16_t* out = cb + (int64_t)bcg * Q * Q;
  const int i0 = 16 * it;
  const int nks = (N + 31) / 32;
  const int njt = min(kCbTiles, Q / 16 - jt0);
  // every operand load is issued before the first MFMA: one memory latency
  // per wave.  C^T operand: lane holds C[i0 + r][32 ks + 8 gq .. + 7], B
  // operand of tile j: B[16 (jt0 + j) + r][same n] (zero past N; tiles
  // above the diagonal are not loaded)
  u32x4_t cf[NKS], bf[kCbTiles][NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int n = 32 * ks + 8 * gq;
    const bool live = ks < nks && n < N && jt0 <= it;
    cf[ks] = live ? *reinterpret_cast<const u32x4_t*>(Cc + (int64_t)(i0 + r) * N + n)
                  : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < kCbTiles; ++j)
      bf[j][ks] = live && j < njt && jt0 + j <= it
                      ? *reinterpret_cast<const u32x4_t*>(Bc + (int64_t)(16 * (jt0 + j) + r) * N + n)
                      : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kCbTiles; ++j) {
    if (j >= njt) continue;
    const int jt = jt0 + j;
    uint16_t* orow = out + (int64_t)(i0 + r) * Q + 16 * jt + 4 * gq;
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (jt <= it) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        if (ks < nks) acc = mfma16t<F16>(bf[j][ks], cf[ks], acc);  // D[j][i] = sum_n B[j][n] C[i][n]
      // lane holds cb[i0 + r][16 jt + 4 gq + e]; the diagonal tile keeps j <= i
      if (jt == it) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * gq + e > r) acc[e] = 0.f;
      }
    }
    *reinterpret_cast<u32x2_t*>(orow) =
        u32x2_t{pack2<F16>(acc[0], acc[1]), pack2<F16>(acc[2], acc[3])};
  }
}

template <bool F16, int NKS>
__global__ void __launch_bounds__(64) ssd_cb_kernel(const uint16_t* __restrict__ Bm,
                                                    const uint16_t* __restrict__ Cm,
                                                    uint16_t* __restrict__ cb, int nc, int G,
                                                    int L, int Q, int N) {
  cb_tiles<F16, NKS>(Bm, Cm, cb, nc, G, L, Q, N, blockIdx.x, blockIdx.y, blockIdx.z, threadIdx.x);
}

// The prologue's first two stages in one launch: they are independent (cb
// does not use dA_cumsum), so the cumsum rows -- the first ncum blocks,
// dispatched first -- run beside the cb tiles instead of ahead of them.
struct CumsumCbParams {
  const float* dt;
  const float* A;
  float* dA;
  const uint16_t* B;
  const uint16_t* C;
  uint16_t* cb;
  int H, nc, G, L, Q, N, per_lane;
  int ncum, nbcg, nit;   // cumsum rows; cb chunks and row bands
};

template <bool F16, int NKS>
__global__ void __launch_bounds__(64) ssd_cumsum_cb_kernel(CumsumCbParams p) {
  const int id = blockIdx.x;
  if (id < p.ncum) {
    cumsum_row(p.dt, p.A, p.dA, p.H, p.nc, p.Q, p.per_lane, id, threadIdx.x);
    return;
  }
  const int k = id - p.ncum;   // the cb grid's (x, y, z) in its dispatch order, x fastest
  cb_tiles<F16, NKS>(p.B, p.C, p.cb, p.nc, p.G, p.L, p.Q, p.N, k % p.nbcg, (k / p.nbcg) % p.nit,
                     k / (p.nbcg * p.nit), threadIdx.x);
}

// ---------------------------------------------------------------------------
// chunk states + state passing -> prev_states_T
// ---------------------------------------------------------------------------
constexpr int kSsdQmax = 512, kSsdPmax = 256, kSsdNmax = 256, kSsdNB = 64, kSsdWaves = 8;
constexpr int kSsdStageMax = 36 * 1024;      // bytes per pipeline stage
constexpr int kSsdRing = 136 * 1024;         // LDS for the stage ring (four 34 KB stages)
constexpr int kSsdNSMax = 8;                 // stages at most
constexpr int kSsdMaxLpw = 5;                // DMA copies per wave per unit at most

// A chunk is processed in units of QS keys (QS divides Q; a chunk whose Q
// is not a multiple of 32 is one unit zero-weighted up to QSP rows).  Unit u
// lives in LDS stage u % NS: x rows [QSP][P] | B rows [QSP][nb] | dA, dt
// (QSP floats each, 1 KB) | dA[c, Q-4 .. Q-1] of the unit's chunk (1 KB slot).
// The WIDE form (P = 64, nb = 64, Q a multiple of 256) takes 256-key units
// in two 67 KB stages: x 32 KB | B 32 KB | dA 1 KB | dt 1 KB | dA tail 1 KB.
struct SsdStateParams {
  const uint16_t* x;
  const float* dt;
  const float* dA;
  const uint16_t* B;
  float* prevT;
  int H, G, nc, Q, P, N, nb;
  int QS, QSP, upc;          // keys per unit, LDS rows per unit, units per chunk
  int xbytes, bbytes;        // per stage
  int ninstr, lpw;           // DMA copies per unit; the most any wave issues
  int ns;                    // stages in the ring (3 .. 8; 2 in the WIDE form)
};

// MODE 0: tile t of wave w is w + 8 t, each with its own p tile.
// MODE 1: P / 16 divides the wave count, so all tiles of a wave share one p
//         tile and the w-scaled x operand is built once per k step.
// MODE 2: P / 16 is half the wave count: waves w and w + P/16 own the same
//         tiles (p tile w % (P/16), every n tile) and split the k steps
//         between them (even / odd), so each scaled x operand is built once
//         per workgroup; at each chunk start the odd wave hands its partial
//         sums to the even wave through LDS, which stores prev(c).  The
//         host picks MODE 2 only for P = 64 (four p tiles) with nb = 16 TPW,
//         so both are compile-time constants there.
// WIDE (MODE 2, TPW 4, QS = 256): the unit layout and every wave's DMA
//         slots are compile-time constants; one wait, barrier, w_c build and
//         prev hand-over per 256 keys instead of two.
template <int TPW, int MODE, bool F16, bool WIDE = false>
__global__ void __launch_bounds__(64 * kSsdWaves) ssd_state_kernel(SsdStateParams p) {
  static_assert(!WIDE || (MODE == 2 && TPW == 4), "256-key units: P = 64, nb = 64 only");
  __shared__ __attribute__((aligned(1024))) char smem[kSsdRing];
  __shared__ __attribute__((aligned(16))) float s_w[kSsdWaves][WIDE ? 256 : 128];
  __shared__ f32x4_t s_x[MODE == 2 ? (kSsdWaves / 2) * TPW * 64 : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, gq = lane >> 4, a4 = r >> 2, c4 = r & 3;
  const int bh = blockIdx.x, nblk = blockIdx.y;
  const int H = p.H, Q = p.Q, N = p.N, nc = p.nc;
  const int P = MODE == 2 ? 16 * (kSsdWaves / 2) : p.P, nb = MODE == 2 ? 16 * TPW : p.nb;
  const int b = bh / H, h = bh % H, g = h / (H / p.G);
  const int n0 = nblk * nb;
  const int L = nc * Q;
  const int XR = P * 2, BR = nb * 2;
  const int QS = WIDE ? 256 : p.QS, QSP = WIDE ? 256 : p.QSP, upc = p.upc, nu = nc * upc;
  const int xbytes = WIDE ? QSP * P * 2 : p.xbytes, bbytes = WIDE ? QSP * nb * 2 : p.bbytes;
  const int stage_bytes = xbytes + bbytes + (WIDE ? 3072 : 2048);
  const int xinstr = xbytes / 1024, binstr = bbytes / 1024;
  const int ptiles = P / 16, tiles = ptiles * (nb / 16);
  // side region of a stage: dA of the unit's keys from float 0, dt from
  // float DTO, dA[c, Q-4 .. Q-1] from float 2 DTO
  constexpr int DTO = WIDE ? 256 : 128;

  const uint16_t* xg = p.x + (int64_t)bh * L * P;
  const uint16_t* bgp = p.B + (int64_t)(b * p.G + g) * L * N + n0;
  const float* dAg = p.dA + (int64_t)bh * nc * Q;
  const float* dtg = p.dt + (int64_t)bh * nc * Q;
  lds_char_t* const sm = (lds_char_t*)smem;
  const int NS = WIDE ? 2 : p.ns;

  // ---- DMA of unit u into stage s; rows past the unit's keys are clamped
  // (their weight is forced to zero).  Copy j of the unit belongs to wave
  // j % 8, so wave w issues nlw = ceil((ninstr - w) / 8) copies per unit,
  // its slots i = 0 .. nlw-1 (j = w + 8 i).  A slot's source offset within
  // the unit and its LDS offset within the stage are the same for every
  // unit: computed once here.
  const int ninstr = WIDE ? xinstr + binstr + 3 : p.ninstr;
  const int nlw = (ninstr - wave + kSsdWaves - 1) / kSsdWaves;
  constexpr int LPW = WIDE ? 8 : kSsdMaxLpw;
  int goff[LPW], loff[LPW], kind[LPW];  // kind: 0 x, 1 B, 2 dA|dt, 3 dA tail
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int j = wave + kSsdWaves * i;
    if (j < xinstr) {
      // LDS slot (row, chunk) of the [QSP][P] unit holds global chunk
      // chunk ^ tr_swz(row): transposed reads of 8 rows then hit distinct banks
      const int e = (j * 64 + lane) * 8;          // element offset in the [QSP][P] unit
      const int row = e / P, cc = (e % P) / 8;
      goff[i] = min(row, QS - 1) * P + (cc ^ tr_swz(row, XR)) * 8;
      loff[i] = j * 1024;
      kind[i] = 0;
    } else if (j < xinstr + binstr) {
      const int idx = (j - xinstr) * 64 + lane;
      const int row = idx / (nb / 8), cc = idx % (nb / 8);
      goff[i] = min(row, QS - 1) * N + (cc ^ tr_swz(row, BR)) * 8;
      loff[i] = xbytes + (j - xinstr) * 1024;
      kind[i] = 1;
    } else {
      goff[i] = min(4 * (lane & 31), QS - 4);
      loff[i] = xbytes + bbytes + (j == xinstr + binstr ? 0 : 1024);
      kind[i] = j == xinstr + binstr ? 2 : 3;
    }
  }
  // slots [i0, i1) of unit u
  auto issue = [&](int s, int u, int i0, int i1) {
    const int c = u / upc, ko = (u % upc) * QS;
    const int64_t key0 = (int64_t)c * Q + ko;   // first key of the unit within (b, h)
    const uint32_t base = lds_addr(sm + s * stage_bytes);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      if (i < i0 || i >= i1) continue;
      const uint32_t la = base + loff[i];
      if (kind[i] == 0) dma_load16(xg + key0 * P + goff[i], la);
      else if (kind[i] == 1) dma_load16(bgp + key0 * N + goff[i], la);
      else if (kind[i] == 2) dma_load16((lane >> 5 ? dtg : dAg) + key0 + goff[i], la);
      else dma_load16(dAg + (int64_t)c * Q + Q - 4, la);
    }
  };
  // 256-key units (P = 64, nb = 64): 32 x copies, 32 B copies and 3 side
  // copies (dA, dt, dA tail), copy j of each kind on wave j % 8, so every
  // wave's slots are compile-time: x slots 0..3 (part 0), B slots 4..7 and
  // waves 0..2 one side copy (part 1).  Source: the unit's base in SGPRs
  // plus the lane's 32-bit byte offset (kept from the setup above: goff is
  // an element offset there).
  auto issue_wide = [&](int s, int u, int part) {
    const int c = u / upc;
    const int64_t key0 = (int64_t)c * Q + (u % upc) * 256;
    const uint32_t base = lds_addr(sm + s * stage_bytes);
    if (part == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dma_load16_s(2u * goff[i], xg + key0 * P, base + (wave + kSsdWaves * i) * 1024);
    } else {
#pragma unroll
      for (int i = 4; i < 8; ++i)
        dma_load16_s(2u * goff[i], bgp + key0 * N, base + xbytes + (wave + kSsdWaves * (i - 4)) * 1024);
      const uint32_t la = base + xbytes + bbytes + wave * 1024;
      if (wave == 2) dma_load16_s(0u, dAg + (int64_t)c * Q + Q - 4, la);
      else if (wave < 2) dma_load16_s(16u * lane, (wave ? dtg : dAg) + key0, la);
    }
  };
  auto wait_units = [&](int younger, int stores) {
    // two stages: the awaited unit's copies are this wave's youngest
    // (issued after its prev stores), so the wait takes everything
    const int n = WIDE ? 0 : younger * nlw + stores;
    switch (n) {
      case 0: LOOM_WAIT_VMCNT(0); break;
      case 1: LOOM_WAIT_VMCNT(1); break;
      case 2: LOOM_WAIT_VMCNT(2); break;
      case 3: LOOM_WAIT_VMCNT(3); break;
      case 4: LOOM_WAIT_VMCNT(4); break;
      case 5: LOOM_WAIT_VMCNT(5); break;
      case 6: LOOM_WAIT_VMCNT(6); break;
      case 7: LOOM_WAIT_VMCNT(7); break;
      case 8: LOOM_WAIT_VMCNT(8); break;
      case 9: LOOM_WAIT_VMCNT(9); break;
      case 10: LOOM_WAIT_VMCNT(10); break;
      case 11: LOOM_WAIT_VMCNT(11); break;
      case 12: LOOM_WAIT_VMCNT(12); break;
      case 13: LOOM_WAIT_VMCNT(13); break;
      case 14: LOOM_WAIT_VMCNT(14); break;
      case 15: LOOM_WAIT_VMCNT(15); break;
      case 16: LOOM_WAIT_VMCNT(16); break;
      case 17: LOOM_WAIT_VMCNT(17); break;
      case 18: LOOM_WAIT_VMCNT(18); break;
      case 19: LOOM_WAIT_VMCNT(19); break;
      case 20: LOOM_WAIT_VMCNT(20); break;
      case 21: LOOM_WAIT_VMCNT(21); break;
      case 22: LOOM_WAIT_VMCNT(22); break;
      case 23: LOOM_WAIT_VMCNT(23); break;
      default: LOOM_WAIT_VMCNT(24); break;
    }
  };

  // running prev_states^T tiles: R[t] is tile (pt, nt) = ((w + 8 t) % ptiles,
  // (w + 8 t) / ptiles) in MODES 0 and 1, (w % ptiles, t) in MODE 2 (there a
  // partial sum over half the k steps); lane holds
  // prev[n0 + 16 nt + r][16 pt + 4 gq + e]
  f32x4_t R[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) R[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // kq: this wave's k-step parity (MODE 2); ntw: tiles it accumulates; nst:
  // prev stores it issues per chunk
  const int kq = MODE == 2 ? wave / ptiles : 0;
  const int ntw = MODE == 2 ? TPW : min(TPW, max(0, (tiles - wave + kSsdWaves - 1) / kSsdWaves));
  const int nst = MODE == 2 ? (kq == 0 ? TPW : 0) : ntw;
  // w_c[k] = exp(dA[c, Q-1] - dA[c, k]) dt[c, k] of the current unit (zero
  // past its QS keys), one copy per wave in s_w[wave]: a wave writes and
  // reads only its own row, so no barrier is involved, and its LDS
  // operations execute in order, so its reads of the row see its writes
  // without a wait.  dAs: the stage's dA (keys 0..127), dt (128..255) and
  // dA[c, Q-4 .. Q-1] (256..259); every one of the 256 was written by the
  // unit's DMA (keys past QS repeat the last ones).  A wave computes the
  // keys of its own k steps only: in MODE 2 steps kq and kq + 2, one key per
  // lane; otherwise all QSP <= 128 keys, two per lane, both loads issued
  // before either exp.
  float* const sw = s_w[wave];
  const float kLog2e = 1.4426950408889634f;
  auto make_w = [&](const float* dAs) {
    const float last = dAs[2 * DTO + 3];
    if constexpr (WIDE) {
      // 256 keys, every one inside the unit: steps kq + 2 m, m = 0..3, lanes
      // 0-31 taking m = 0 and 2, lanes 32-63 m = 1 and 3
      const int i0 = 32 * (kq + 2 * (lane >> 5)) + (lane & 31), i1 = i0 + 128;
      const float a0 = dAs[i0], t0 = dAs[DTO + i0], a1 = dAs[i1], t1 = dAs[DTO + i1];
      sw[i0] = fast_exp2((last - a0) * kLog2e) * t0;
      sw[i1] = fast_exp2((last - a1) * kLog2e) * t1;
    } else if constexpr (MODE == 2) {
      const int s = kq + 2 * (lane >> 5), i = 32 * s + (lane & 31);
      const float a = dAs[i], t = dAs[128 + i];
      if (32 * s < QSP) sw[i] = i < QS ? fast_exp2((last - a) * kLog2e) * t : 0.f;
    } else {
      const int i0 = lane, i1 = lane + 64;
      const float a0 = dAs[i0], t0 = dAs[128 + i0], a1 = dAs[i1], t1 = dAs[128 + i1];
      if (i0 < QSP) sw[i0] = i0 < QS ? fast_exp2((last - a0) * kLog2e) * t0 : 0.f;
      if (i1 < QSP) sw[i1] = i1 < QS ? fast_exp2((last - a1) * kLog2e) * t1 : 0.f;
    }
  };

  // x^T operand (keys k0 + 0..3 from x0, k0 + 16..19 from x1) scaled by w
  // and split into bf16 hi + lo: the products keep ~16 significant bits
  auto scale_x = [&](const u32x2_t& x0, const u32x2_t& x1, const f32x4_t& w0, const f32x4_t& w1,
                     u32x4_t& vh, u32x4_t& vl) {
    const float v[8] = {lo16<F16>(x0[0]) * w0[0], hi16<F16>(x0[0]) * w0[1],
                        lo16<F16>(x0[1]) * w0[2], hi16<F16>(x0[1]) * w0[3],
                        lo16<F16>(x1[0]) * w1[0], hi16<F16>(x1[0]) * w1[1],
                        lo16<F16>(x1[1]) * w1[2], hi16<F16>(x1[1]) * w1[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vh[e] = pack2<F16>(v[2 * e], v[2 * e + 1]);
      vl[e] = pack2<F16>(v[2 * e] - lo16<F16>(vh[e]), v[2 * e + 1] - hi16<F16>(vh[e]));
    }
  };
  // MFMA operands of one 32-key step: x^T of p tile pt, w, and B of the
  // wave's n tiles (n = 16 nt + r); tiles past the wave's count read tile
  // tiles-1 (in range, results unused)
  struct Ops {
    u32x2_t x0, x1;
    f32x4_t w0, w1;
    u32x2_t b0[TPW], b1[TPW];
  };
  // Byte offset, within a stage's x (row width XR) or B (BR) rows, of the
  // operand this lane reads for p or n tile `tile` at k step 0: row
  // kk = 4 gq + a4, 16-byte chunk 2 tile + c4/2 under the row's swizzle.
  // Step ks reads 32 ks rows further on, with the same swizzle: tr_swz reads
  // bits 0..2 of the row only, so rows kk, kk + 16 and kk + 32 ks share it.
  const int kk = 4 * gq + a4;
  auto op_off = [&](int tile, int rb) {
    return kk * rb + ((2 * tile + (c4 >> 1)) ^ tr_swz(kk, rb)) * 16 + (c4 & 1) * 8;
  };
  // the offsets of the wave's own tiles (MODES 1 and 2), computed once
  int xo = 0, bo[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) bo[t] = 0;
  if constexpr (MODE >= 1) {
    xo = op_off(wave % ptiles, XR);
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      bo[t] = op_off(MODE == 2 ? t : min(wave + kSsdWaves * t, tiles - 1) / ptiles, BR);
  }
  auto load_ops = [&](const lds_char_t* xs, const lds_char_t* bs, int ks, Ops& o) {
    const int k0 = 32 * ks + 4 * gq;          // this lane's keys: k0 + 0..3, k0 + 16..19
    const lds_char_t* qx = xs + 32 * ks * XR + xo;
    o.x0 = lds_read_tr16(qx);
    o.x1 = lds_read_tr16(qx + 16 * XR);
    o.w0 = *reinterpret_cast<const f32x4_t*>(sw + k0);
    o.w1 = *reinterpret_cast<const f32x4_t*>(sw + k0 + 16);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const lds_char_t* qb = bs + 32 * ks * BR + bo[t];
      o.b0[t] = lds_read_tr16(qb);
      o.b1[t] = lds_read_tr16(qb + 16 * BR);
    }
  };

  auto compute = [&](int s, int u) {
    const int c = u / upc, part = u % upc;
    const lds_char_t* xs = sm + s * stage_bytes;
    const lds_char_t* bs = xs + xbytes;
    const float* dAs = reinterpret_cast<const float*>(smem + s * stage_bytes + xbytes + bbytes);
    // the DMA of unit u+NS-1 (into the stage unit u-1 used) is issued in two
    // halves between this unit's steps, so the address units work through
    // it while the waves compute
    const bool pre = u + NS - 1 < nu;
    const int sn = (u + NS - 1) % NS, un = u + NS - 1, half = (nlw + 1) / 2;
    make_w(dAs);
    lds_order();   // the w row's float stores before its f32x4 reads below
    if (part == 0) {
      // prev(c) out, then R = exp(dA[c, Q-1]) R; states(c) accumulate below
      const float decay = fast_exp2(dAs[2 * DTO + 3] * kLog2e);
      float* outc = p.prevT + (((int64_t)(b * nc + c) * H + h) * N + n0) * P;
      if constexpr (MODE == 2) {
        const int pt = wave % ptiles;
        f32x4_t* xch = s_x + pt * TPW * 64 + lane;
        if (kq == 1) {
#pragma unroll
          for (int t = 0; t < TPW; ++t) xch[t * 64] = R[t];
        }
        LOOM_WAIT_LGKM0();
        barrier_nofence();
        if (kq == 0) {
#pragma unroll
          for (int t = 0; t < TPW; ++t)
            *reinterpret_cast<f32x4_t*>(outc + (int64_t)(16 * t + r) * P + 16 * pt + 4 * gq) =
                R[t] + xch[t * 64];
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t) R[t] *= decay;
      } else {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const int tt = wave + kSsdWaves * t;
          if (tt < tiles) {
            const int pt = tt % ptiles, nt = tt / ptiles;
            *reinterpret_cast<f32x4_t*>(outc + (int64_t)(16 * nt + r) * P + 16 * pt + 4 * gq) = R[t];
            R[t] *= decay;
          }
        }
      }
    }
    const int nks = QSP / 32;
    if constexpr (MODE >= 1) {
      // all tiles of the wave share p tile wave % ptiles: one scaled x
      // operand per step (MODE 2: every other step); the next step's
      // operands are read while this step's MFMAs run
      // (two operand sets alternate, so nothing is copied between steps,
      // and the last step reads nothing ahead)
      constexpr int KSTEP = MODE == 2 ? 2 : 1;
      auto step = [&](const Ops& o) {
        u32x4_t xh, xl;
        scale_x(o.x0, o.x1, o.w0, o.w1, xh, xl);
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          if (t < ntw) {
            const u32x4_t bf = u32x4_t{o.b0[t][0], o.b0[t][1], o.b1[t][0], o.b1[t][1]};
            R[t] = mfma16t<F16>(xh, bf, R[t]);
            R[t] = mfma16t<F16>(xl, bf, R[t]);
          }
        }
      };
      if (kq < nks) {
        Ops oa, ob;
        load_ops(xs, bs, kq, oa);
        for (int ks = kq; ks < nks; ks += 2 * KSTEP) {
          if (ks + KSTEP < nks) load_ops(xs, bs, ks + KSTEP, ob);
          step(oa);
          if (ks == kq && pre) {
            if constexpr (WIDE) issue_wide(sn, un, 0);
            else issue(sn, un, 0, half);
          }
          if (ks + KSTEP >= nks) break;
          if (ks + 2 * KSTEP < nks) load_ops(xs, bs, ks + 2 * KSTEP, oa);
          step(ob);
        }
      } else if (pre) {
        if constexpr (WIDE) issue_wide(sn, un, 0);
        else issue(sn, un, 0, half);
      }
      if (pre) {
        if constexpr (WIDE) issue_wide(sn, un, 1);
        else issue(sn, un, half, nlw);
      }
    } else {
      if (pre) issue(sn, un, 0, nlw);
      for (int ks = 0; ks < nks; ++ks) {
        const int k0 = 32 * ks + 4 * gq;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const int tt = wave + kSsdWaves * t;
          if (tt < tiles) {
            const int pt = tt % ptiles, nt = tt / ptiles;
            const lds_char_t* qx = xs + 32 * ks * XR + op_off(pt, XR);
            u32x4_t xh, xl;
            scale_x(lds_read_tr16(qx), lds_read_tr16(qx + 16 * XR),
                    *reinterpret_cast<const f32x4_t*>(sw + k0),
                    *reinterpret_cast<const f32x4_t*>(sw + k0 + 16), xh, xl);
            const lds_char_t* qb = bs + 32 * ks * BR + op_off(nt, BR);
            const u32x2_t blo = lds_read_tr16(qb), bhi = lds_read_tr16(qb + 16 * BR);
            const u32x4_t bf = u32x4_t{blo[0], blo[1], bhi[0], bhi[1]};
            R[t] = mfma16t<F16>(xh, bf, R[t]);
            R[t] = mfma16t<F16>(xl, bf, R[t]);
          }
        }
      }
    }
  };

  // ---- pipeline: units issued NS-1 ahead.  Iteration u waits for unit u
  // only, so NS-1 units are in flight while it waits.  The DMA issued by
  // compute(u), after the barrier of iteration u, reuses the stage of unit
  // u-1, whose reads every wave finished before that barrier.  prev stores
  // issued by compute(u) are younger than unit u+NS-2's DMA, so the next
  // wait (for unit u+1) leaves them outstanding too.
  for (int u = 0; u < NS - 1 && u < nu; ++u) {
    if constexpr (WIDE) {
      issue_wide(u, u, 0);
      issue_wide(u, u, 1);
    } else {
      issue(u, u, 0, nlw);
    }
  }
  int stores = 0;
  for (int u = 0; u < nu; ++u) {
    wait_units(max(0, min(NS - 2, nu - 1 - u)), stores);
    LOOM_WAIT_LGKM0();                        // this wave's reads of unit u-1's stage done
    barrier_nofence();
    compute(u % NS, u);
    stores = (u % upc == 0) ? nst : 0;
  }
}

template <int TPW, bool F16>
void launch_state(const SsdStateParams& p, int mode, int grid_x, int grid_y, hipStream_t st) {
  const dim3 grid((unsigned)grid_x, (unsigned)grid_y), block(64 * kSsdWaves);
  if constexpr (TPW == 4) {
    if (mode == 2 && p.QS == 256) {
      hipLaunchKernelGGL((ssd_state_kernel<4, 2, F16, true>), grid, block, 0, st, p);
      return;
    }
  }
  if (mode == 2)
    hipLaunchKernelGGL((ssd_state_kernel<TPW, 2, F16>), grid, block, 0, st, p);
  else if (mode == 1)
    hipLaunchKernelGGL((ssd_state_kernel<TPW, 1, F16>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((ssd_state_kernel<TPW, 0, F16>), grid, block, 0, st, p);
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
  if (chunk_size > kSsdQmax || headdim > kSsdPmax || dstate > kSsdNmax ||
      (dstate > 32 && dstate % 32))
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: built for chunk_size <= %d, headdim <= %d, dstate <= %d "
                     "(a multiple of 32 above 32)",
                     fn, kSsdQmax, kSsdPmax, kSsdNmax);
  if (!loom_prod_le({batch, nheads, nchunks, chunk_size, headdim}, ((int64_t)1 << 40) - 1) ||
      !loom_prod_le({batch, nchunks, nheads, dstate, headdim}, (int64_t)1 << 40) ||
      !loom_prod_le({batch, ngroups, nchunks, chunk_size, dstate}, (int64_t)1 << 40))
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
  if (!loom_prod_le({batch, nheads, nchunks, chunk_size}, (int64_t)1 << 40) ||
      !loom_prod_le({batch, nheads, nchunks}, 0x7fffffff / 64))
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_chunk_cumsum: problem too large");
  const int per_lane = (int)((chunk_size + 63) / 64);
  if (loom_validate_only()) return loom_ok(err, errlen);
  hipLaunchKernelGGL(ssd_cumsum_kernel, dim3((unsigned)(batch * nheads * nchunks)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(dt),
                     static_cast<const float*>(A), static_cast<float*>(dA_cumsum), (int)nheads,
                     (int)nchunks, (int)chunk_size, per_lane);
  return loom_check_launch(err, errlen, "ssd_chunk_cumsum");
}

}  // extern "C"

namespace {

template <bool F16>
int bmm_chunk_impl(const void* B, const void* C, void* cb, int64_t batch, int64_t nchunks,
                           int64_t ngroups, int64_t chunk_size, int64_t dstate, void* stream,
                           char* err, size_t errlen) {
  if (!B || !C || !cb) return loom_fail(err, errlen, LOOM_EINVAL, "ssd_bmm_chunk: null tensor pointer");
  int rc = check_ssd("ssd_bmm_chunk", batch, nchunks, ngroups, ngroups, chunk_size, 16, dstate,
                     err, errlen);
  if (rc) return rc;
  if (!aligned16(B) || !aligned16(C) || (reinterpret_cast<uintptr_t>(cb) & 7u))
    return loom_fail(err, errlen, LOOM_EINVAL, "ssd_bmm_chunk: B, C 16-byte and cb 8-byte aligned");
  if (loom_validate_only()) return loom_ok(err, errlen);
  const dim3 grid((unsigned)(batch * nchunks * ngroups), (unsigned)(chunk_size / 16),
                  (unsigned)((chunk_size / 16 + kCbTiles - 1) / kCbTiles));
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(B), static_cast<const uint16_t*>(C),
                       static_cast<uint16_t*>(cb), (int)nchunks, (int)ngroups,
                       (int)(nchunks * chunk_size), (int)chunk_size, (int)dstate);
  };
  if (dstate <= 128) launch(ssd_cb_kernel<F16, 4>);
  else launch(ssd_cb_kernel<F16, 8>);
  return loom_check_launch(err, errlen, "ssd_bmm_chunk");
}

template <bool F16>
int state_passing_impl(const void* x, const void* dt, const void* dA_cumsum,
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
  // (and 32 when 64 does not divide dstate; dstate itself up to 32)
  const int nb_cap = headdim <= 128 ? kSsdNB : 32;
  const int nb = dstate <= nb_cap ? (int)dstate : (dstate % nb_cap == 0 ? nb_cap : 32);
  const int ptiles = (int)(headdim / 16), tiles = ptiles * (nb / 16);
  // kernel mode (see ssd_state_kernel) and tiles per wave
  const int mode = kSsdWaves % ptiles ? 0 : (2 * ptiles == kSsdWaves ? 2 : 1);
  const int tpw = mode == 2 ? nb / 16 : (tiles + kSsdWaves - 1) / kSsdWaves;
  if (dstate % nb != 0 || tpw > 4)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "ssd_chunk_state_passing: dstate %lld with headdim %lld not built",
                     (long long)dstate, (long long)headdim);
  SsdStateParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.dt = static_cast<const float*>(dt);
  p.dA = static_cast<const float*>(dA_cumsum);
  p.B = static_cast<const uint16_t*>(B);
  p.prevT = static_cast<float*>(prev_states_T);
  p.H = (int)nheads; p.G = (int)ngroups; p.nc = (int)nchunks; p.Q = (int)chunk_size;
  p.P = (int)headdim; p.N = (int)dstate; p.nb = nb;
  // unit (when the WIDE form does not apply): the largest of 128, 64 and 32
  // keys dividing Q whose stage fits, else the largest other multiple of 16
  // (a unit that is not a multiple of 32 keys is zero-weighted up to the
  // next one)
  // (each unit costs a barrier and a wait, and the copies in flight per
  // workgroup, not the ring depth, bound the stream: 128-key units measured
  // faster than 64-key units with twice the stages); a Q that is not a
  // multiple of 32 is one unit padded to the next 32.  Stages: as many as
  // fit while the wait count stays encodable.
  auto plan = [&](int qs, SsdStateParams& q) {
    q.QS = qs;
    q.QSP = (qs + 31) & ~31;
    q.upc = q.Q / qs;
    q.xbytes = (q.QSP * q.P * 2 + 1023) & ~1023;  // whole 1 KB DMA copies
    q.bbytes = (q.QSP * nb * 2 + 1023) & ~1023;
    q.ninstr = q.xbytes / 1024 + q.bbytes / 1024 + 2;
    q.lpw = (q.ninstr + kSsdWaves - 1) / kSsdWaves;
    if (q.lpw > kSsdMaxLpw) return -1;
    if (q.xbytes + q.bbytes + 2048 > kSsdStageMax) return -1;
    q.ns = std::min(kSsdNSMax, kSsdRing / (q.xbytes + q.bbytes + 2048));
    while (q.ns > 3 && q.lpw * (q.ns - 2) + tpw > 24) --q.ns;
    if (q.ns < 3 || q.lpw * (q.ns - 2) + tpw > 24) return -1;
    return (q.ns - 1) * (q.xbytes + q.bbytes);
  };
  int best = -1;
  // P = 64 with a 64-wide n block and Q a multiple of 256: 256-key units in
  // two 67 KB stages (the kernel's WIDE form, its layout fixed at compile
  // time); one barrier, wait and hand-over per 256 keys instead of two
  if (mode == 2 && tpw == 4 && p.Q % 256 == 0) {
    p.QS = p.QSP = 256;
    p.upc = p.Q / 256;
    p.xbytes = 256 * 64 * 2;
    p.bbytes = 256 * 64 * 2;
    p.ninstr = p.xbytes / 1024 + p.bbytes / 1024 + 3;
    p.lpw = (p.ninstr + kSsdWaves - 1) / kSsdWaves;
    p.ns = 2;
    static_assert(2 * (256 * 64 * 2 * 2 + 3072) <= kSsdRing, "two 256-key stages fit the ring");
    best = 0;
  }
  for (int qs : {128, 64, 32, 112, 96, 80, 48, 16}) {
    if (best >= 0) break;
    if (p.Q % qs) continue;
    SsdStateParams q = p;
    if ((best = plan(qs, q)) >= 0) { p = q; break; }
  }
  if (best < 0 && p.Q % 32 != 0 && p.Q < 128) best = plan(p.Q, p);
  if (best < 0)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "ssd_chunk_state_passing: chunk_size %lld with headdim %lld does not fit "
                     "an LDS stage",
                     (long long)chunk_size, (long long)headdim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int gx = (int)(batch * nheads), gy = (int)(dstate / nb);
  if (loom_validate_only()) return loom_ok(err, errlen);
  if (tpw <= 1) launch_state<1, F16>(p, mode, gx, gy, st);
  else if (tpw <= 2) launch_state<2, F16>(p, mode, gx, gy, st);
  else launch_state<4, F16>(p, mode, gx, gy, st);
  return loom_check_launch(err, errlen, "ssd_chunk_state_passing");
}

template <bool F16>
int prologue_impl(const void* x, const void* dt, const void* A, const void* B,
                          const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                          int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                          int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                          char* err, size_t errlen) {
  int rc = check_ssd("ssd_prologue", batch, nchunks, nheads, ngroups, chunk_size, headdim, dstate,
                     err, errlen);
  if (rc) return rc;
  // the three stages' own checks run first, validate-only, so a shape the
  // last stage rejects (e.g. an LDS plan that does not fit) launches nothing
  auto stages = [&]() {
    int r = loom_hip_ssd_chunk_cumsum(dt, A, dA_cumsum, batch, nchunks, nheads, chunk_size,
                                      stream, err, errlen);
    if (r) return r;
    r = bmm_chunk_impl<F16>(B, C, cb, batch, nchunks, ngroups, chunk_size, dstate, stream, err,
                            errlen);
    if (r) return r;
    return state_passing_impl<F16>(x, dt, dA_cumsum, B, prev_states_T, batch, nchunks, nheads,
                                   ngroups, chunk_size, headdim, dstate, stream, err, errlen);
  };
  bool& vo = loom_validate_only_flag();
  const bool outer = vo;
  vo = true;
  rc = stages();
  vo = outer;
  if (rc || outer) return rc;
  // cumsum and cb in one launch (independent of each other), then the states
  const int64_t ncum = batch * nheads * nchunks, nbcg = batch * nchunks * ngroups;
  const int64_t nit = chunk_size / 16, njz = (nit + kCbTiles - 1) / kCbTiles;
  const int64_t nblocks = ncum + nbcg * nit * njz;
  if (nblocks > 0x7fffffff) return stages();
  CumsumCbParams q{};
  q.dt = static_cast<const float*>(dt);
  q.A = static_cast<const float*>(A);
  q.dA = static_cast<float*>(dA_cumsum);
  q.B = static_cast<const uint16_t*>(B);
  q.C = static_cast<const uint16_t*>(C);
  q.cb = static_cast<uint16_t*>(cb);
  q.H = (int)nheads;
  q.nc = (int)nchunks;
  q.G = (int)ngroups;
  q.L = (int)(nchunks * chunk_size);
  q.Q = (int)chunk_size;
  q.N = (int)dstate;
  q.per_lane = (int)((chunk_size + 63) / 64);
  q.ncum = (int)ncum;
  q.nbcg = (int)nbcg;
  q.nit = (int)nit;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dstate <= 128)
    hipLaunchKernelGGL((ssd_cumsum_cb_kernel<F16, 4>), dim3((unsigned)nblocks), dim3(64), 0, st, q);
  else
    hipLaunchKernelGGL((ssd_cumsum_cb_kernel<F16, 8>), dim3((unsigned)nblocks), dim3(64), 0, st, q);
  rc = loom_check_launch(err, errlen, "ssd_prologue (cumsum and cb)");
  if (rc) return rc;
  return state_passing_impl<F16>(x, dt, dA_cumsum, B, prev_states_T, batch, nchunks, nheads,
                                 ngroups, chunk_size, headdim, dstate, stream, err, errlen);
}

}  // namespace

extern "C" {

int loom_hip_ssd_bmm_chunk(const void* B, const void* C, void* cb, int64_t batch, int64_t nchunks,
                           int64_t ngroups, int64_t chunk_size, int64_t dstate, void* stream,
                           char* err, size_t errlen) {
  return bmm_chunk_impl<false>(B, C, cb, batch, nchunks, ngroups, chunk_size, dstate, stream, err,
                               errlen);
}
int loom_hip_ssd_bmm_chunk_f16(const void* B, const void* C, void* cb, int64_t batch,
                               int64_t nchunks, int64_t ngroups, int64_t chunk_size,
                               int64_t dstate, void* stream, char* err, size_t errlen) {
  return bmm_chunk_impl<true>(B, C, cb, batch, nchunks, ngroups, chunk_size, dstate, stream, err,
                              errlen);
}
int loom_hip_ssd_chunk_state_passing(const void* x, const void* dt, const void* dA_cumsum,
                                     const void* B, void* prev_states_T, int64_t batch,
                                     int64_t nchunks, int64_t nheads, int64_t ngroups,
                                     int64_t chunk_size, int64_t headdim, int64_t dstate,
                                     void* stream, char* err, size_t errlen) {
  return state_passing_impl<false>(x, dt, dA_cumsum, B, prev_states_T, batch, nchunks, nheads,
                                   ngroups, chunk_size, headdim, dstate, stream, err, errlen);
}
int loom_hip_ssd_chunk_state_passing_f16(const void* x, const void* dt, const void* dA_cumsum,
                                         const void* B, void* prev_states_T, int64_t batch,
                                         int64_t nchunks, int64_t nheads, int64_t ngroups,
                                         int64_t chunk_size, int64_t headdim, int64_t dstate,
                                         void* stream, char* err, size_t errlen) {
  return state_passing_impl<true>(x, dt, dA_cumsum, B, prev_states_T, batch, nchunks, nheads,
                                  ngroups, chunk_size, headdim, dstate, stream, err, errlen);
}
int loom_hip_ssd_prologue(const void* x, const void* dt, const void* A, const void* B,
                          const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                          int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                          int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                          char* err, size_t errlen) {
  return prologue_impl<false>(x, dt, A, B, C, dA_cumsum, cb, prev_states_T, batch, nchunks,
                              nheads, ngroups, chunk_size, headdim, dstate, stream, err, errlen);
}
int loom_hip_ssd_prologue_f16(const void* x, const void* dt, const void* A, const void* B,
                              const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                              int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                              int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                              char* err, size_t errlen) {
  return prologue_impl<true>(x, dt, A, B, C, dA_cumsum, cb, prev_states_T, batch, nchunks,
                             nheads, ngroups, chunk_size, headdim, dstate, stream, err, errlen);
}

}  // extern "C"
