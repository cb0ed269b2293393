// mamba.hip -- @helion_mamba2_chunk_scan_kernel (Mamba-2 SSD chunk scan) on gfx950.
//
// Reference: examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4-126,
// fused form examples/mamba_chunk_scan/IR/01_tensor_canonicalized.mlir:55-106.
// Shapes: cb [b,c,G,Q,Q] bf16, x [b,H,L,P] bf16, dt and dA_cumsum [b,H,c,Q]
// fp32, C [b,G,L,N] bf16, D [H] fp32, prev_states_T [b,c,H,N,P] fp32,
// out [b,H,L,P] bf16, L = c*Q, group g = h / (H/G).  For every (b,h,c):
//   out[m,p] = exp(dA[m]) * sum_n C[m,n] prevT[n,p]                 (:46-56)
//            + sum_{k<=m} cb[m,k] exp(dA[m]-dA[k]) dt[k] x[k,p]     (:57-104)
//            + D[h] x[m,p]                                          (:105-121)
// The k <= m mask is the Mamba-2 intra-chunk causal mask, applied with a
// select; the reference loop has none and would overflow exp() there.
//
// gfx950 mapping.  One workgroup per (b, h, c, m-tile, p-tile): 8 waves when
// the m-tile holds 8 or more 16-row tiles, else 4; logical ids are ordered
// (b, c, h, tile) and remapped so that each XCD owns whole (b, c) groups:
// the heads that share cb and C then run together on one L2.  The 8-wave
// form fits 128 VGPRs, so two of its workgroups (67 KB of LDS each at
// tile_n 64) give every SIMD four waves to switch between while one waits
// on its row loads or LDS reads (BASELINE shape: 93.8 -> 83.0 us against two
// 4-wave workgroups per CU).  Per workgroup:
//   - x[k, p] (k < m-tile end) is copied to LDS transposed (xT [p][k]) by
//     8x8 register transposes: the B operand of W . x; xT and pT rows XOR
//     their 16-byte chunk index with row & 15, so the 16 rows a ds_read_b128
//     pass reads (every row at the same offset of the 256-byte bank window)
//     hit distinct banks;
//   - prevT[n, p] (fp32) is split into bf16 hi + lo halves, transposed into
//     LDS (pT [p][n]): the B operand of C . prevT, so the state term keeps
//     about 16 mantissa bits;
//   - C rows and cb rows are read from global straight into A-operand
//     registers (k / n contiguous), W = cb * exp2((dA_m - dA_k) log2 e) * dt_k
//     is formed in fp32 registers, masked, and split into bf16 hi + lo
//     operands (a single bf16 rounding of W costs ~2^-9 per term, which
//     summed over a 256-long chunk exceeds the 2e-2 output tolerance);
//   - 16-row m tiles are dealt to the waves in a snake order so the causal
//     triangle costs every wave the same;
//   - the MFMAs compute out^T tiles, so each lane holds four consecutive
//     columns of one output row: the exp(dA[m]) scale is one factor per lane
//     and results are stored as 8-byte writes straight from registers;
//   - D x is folded into the diagonal of W (W[m, m] += D[h]).
#include "common.h"

namespace {

constexpr int kQmax = 256;   // chunk length of the default build
constexpr int kNmax = 128;   // state size of the default build
// The long-chunk build (4 waves, one workgroup per CU: 134 KB of LDS at
// tile_n 64) takes chunks up to 512 and states up to 256 wide.
constexpr int kQbig = 512, kNbig = 256;
constexpr int kMTileMax = 256;   // rows of the largest built m-tile
// upper_bound of the example's tile_k symbol
// (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:3)
constexpr int64_t kMambaTileKBound = 8192;

struct MambaParams {
  const uint16_t* cb;
  const uint16_t* x;
  const void* dt;      // fp32, or f16 in the f16 variant
  const void* dA;      // fp32 / f16
  const uint16_t* C;
  const void* Dh;      // fp32 / f16
  const void* prevT;   // fp32 / f16
  uint16_t* out;
  int Bb, nc, H, G, Q, P, N;
  int tile_m, tile_n, nmt, npt;
  int cus;             // CUs of the launch's device (0: unknown)
};

// Element i of a side tensor (dt, dA_cumsum, D, prev_states_T) as fp32: fp32
// in the bf16 variant, f16 -- the reference's own type
// (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4) -- in the f16
// variant.  The widening is exact.
template <bool F16>
LOOM_DEV float side_at(const void* __restrict__ t, int64_t i) {
  if constexpr (F16)
    return (float)reinterpret_cast<const _Float16* __restrict__>(t)[i];
  else
    return reinterpret_cast<const float* __restrict__>(t)[i];
}

// PT: p tiles of 16 per workgroup (tile_n = 16 PT); F16: f16 elements;
// kWaves: 4 or 8 waves (the 8-wave form is held to 128 VGPRs: four waves per
// SIMD); QM, NM: the longest chunk and the widest state it is built for
template <int PT, bool F16, int kWaves, int QM = kQmax, int NM = kNmax>
__global__ void __launch_bounds__(64 * kWaves, kWaves == 8 ? 4 : 1)
    mamba_chunk_scan_kernel(MambaParams p) {
  static_assert(QM % 128 == 0 && NM % 128 == 0, "xT and pT rows: whole 256-byte bank windows");
  constexpr int TN = 16 * PT;
  constexpr int XROW = QM / 8;   // 16-byte chunks per xT row
  constexpr int PROW = NM / 8;   // 16-byte chunks per pT row
  // LDS sized to the workgroup's TN columns: narrower tiles leave room for
  // more workgroups per CU (tile_n 16: 226.6 -> 179.2 us at the BASELINE
  // shape, against the 64-column size for every tile)
  __shared__ u32x4_t xT[TN * XROW];           // [p][k]
  __shared__ u32x4_t pT[2][TN * PROW];        // hi, lo: [p][n]
  __shared__ __attribute__((aligned(16))) float s_dA[QM], s_dt[QM], s_U[QM];
  // per wave: 8 output rows of a 64-column tile (8 x 128 bytes), staged for
  // whole-row stores
  __shared__ u32x4_t ostage[PT == 4 ? kWaves * 64 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rr = lane & 15, g4 = lane >> 4;
  // Two 8-wave workgroups share a CU, and the dispatcher gives blocks
  // 0 .. cus-1 every CU's first slot and cus .. 2 cus-1 the second.  The
  // second starts ~1 us (2048 clocks) later, so the pair's staging bursts
  // (every load of x and prev_states at once) do not coincide, in the first
  // round or -- each finishing workgroup being replaced -- in later ones
  // (BASELINE shape 82.7 -> 80.0 us; a 4x longer delay gains the same).
  if constexpr (kWaves == 8) {
    if ((int)blockIdx.x >= p.cus && (int)blockIdx.x < 2 * p.cus) __builtin_amdgcn_s_sleep(32);
  }
  const int Q = p.Q, P = p.P, N = p.N, H = p.H;
  const int L = p.nc * Q;

  // ---- logical id -> (b, c, h, m-tile, p-tile)
  const int ntile = p.nmt * p.npt;
  const int nblocks = p.Bb * p.nc * H * ntile;
  int id = xcd_remap(blockIdx.x, nblocks);
  const int tile = id % ntile;
  id /= ntile;
  const int h = id % H;
  id /= H;
  const int c = id % p.nc;
  const int b = id / p.nc;
  const int mt = tile / p.npt, ptl = tile % p.npt;
  const int m0 = mt * p.tile_m;
  const int mend = min(Q, m0 + p.tile_m);
  const int p0 = ptl * TN;
  const int grp = h / (H / p.G);

  const uint16_t* __restrict__ xg = p.x + ((int64_t)(b * H + h) * L + (int64_t)c * Q) * P;
  const uint16_t* __restrict__ Cg = p.C + ((int64_t)(b * p.G + grp) * L + (int64_t)c * Q) * N;
  const uint16_t* __restrict__ cbg = p.cb + ((int64_t)(b * p.nc + c) * p.G + grp) * Q * Q;
  const int64_t pv0 = ((int64_t)(b * p.nc + c) * H + h) * N * P;   // prevT element offset
  const float* __restrict__ pvg = reinterpret_cast<const float*>(p.prevT) + pv0;        // bf16 form
  const uint16_t* __restrict__ pvh = reinterpret_cast<const uint16_t*>(p.prevT) + pv0;  // f16 form
  const int64_t sidx = ((int64_t)(b * H + h) * p.nc + c) * Q;

  const float Dh = side_at<F16>(p.Dh, h);
  const int nmt16 = (mend - m0 + 15) / 16;  // 16-row tiles of this workgroup
  constexpr int MAXT = kMTileMax / 16 / kWaves;  // tiles per wave at most
  constexpr int NSN = NM / 32;                   // state-term steps at most
  constexpr int NKS = QM / 32;                   // intra-chunk steps at most
  // snake deal of 16-row tiles: slot ti of wave w is tile 4 ti + (w or 3 - w)
  auto tile_of = [&](int ti) {
    return kWaves * ti + ((ti & 1) ? (kWaves - 1 - wave) : wave);
  };
  // C and cb rows come straight from global memory as MFMA operands.  A
  // tile's C rows are loaded while the previous tile computes (two register
  // sets); so are its cb rows with 4 waves, while with 8 waves (128 VGPRs)
  // they are loaded at the tile's start, behind its state term's MFMAs.
  // Buffer loads read rows past the chunk as zeros.
  const rsrc_t rC = make_rsrc(Cg, (uint32_t)(Q * N * 2));
  const rsrc_t rCB = make_rsrc(cbg, (uint32_t)(Q * Q * 2));
  constexpr bool kCbAhead = kWaves == 4 && QM == kQmax;   // 64 more VGPRs in the long build
  struct CRows {
    u32x4_t c[NSN];
  };
  struct BRows {
    u32x4_t cb[NKS];
  };
  // Every load is issued, unneeded ones with an offset past the
  // descriptor's range (zeros, no memory access): the compiler can then
  // count the loads younger than the ones it waits for, where a
  // conditional load makes it wait for all of them, prefetch included.
  constexpr uint32_t kNone = 0x7ffffff0u;
  auto fetch_c = [&](int ti, CRows& rw) {
    const int am = m0 + 16 * tile_of(ti) + rr;
#pragma unroll
    for (int ns = 0; ns < NSN; ++ns)
      rw.c[ns] = buf_load16(rC, ns * 32 < N ? (uint32_t)(am * N + ns * 32 + g4 * 8) * 2 : kNone);
  };
  auto fetch_cb = [&](int ti, BRows& rw) {
    const int mrow0 = m0 + 16 * tile_of(ti);
    const int am = mrow0 + rr;
    const int kend = min(mrow0 + 16, Q);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      rw.cb[ks] = buf_load16(rCB, ks * 32 < kend ? (uint32_t)(am * Q + ks * 32 + g4 * 8) * 2 : kNone);
  };

  // The MFMAs compute out^T tiles (x^T / prevT^T as the row operand, W / C
  // as the column operand): lane (rr, g4) of tile (ti, pt) accumulates
  // out[m = mrow0 + rr][p = 16 pt + 4 g4 + i], four consecutive columns.
  uint16_t* og = p.out + ((int64_t)(b * H + h) * L + (int64_t)c * Q) * P;
  CRows cbuf[2];
  BRows bbuf[kCbAhead ? 2 : 1];
  // the first tile's C rows (and, with 4 waves, its cb rows) are loaded
  // before the staging loads, so their latency overlaps the staging instead
  // of following it (BASELINE shape 81.4 -> 78.1 us; the 8-wave form's cb
  // rows as well would spill at 128 VGPRs)
  fetch_c(0, cbuf[0]);
  if constexpr (kCbAhead) fetch_cb(0, bbuf[0]);
  // ---- staging: every global load first, then conversions and LDS stores.
  // One 8x8 block of x per thread (k-chunk fastest; k rounded up to the
  // 32-deep MFMA step, rows past the chunk zero-filled); half an 8x8 block
  // of prevT (rows n = 8 p_nc + 0..7, columns p = 8 p_pc + 4 p_h + 0..3) for
  // each of the first 2*nch*pch threads, from thread 256 on with 8 waves so
  // no thread stages both; one dA and dt value per thread.  The long build
  // has more blocks and keys than threads and stages them in rounds (x
  // block tid + 256 r, and so on); the default build fits one round.
  const int kch = ((mend + 31) / 32) * 4, pch = TN / 8;
  const int nch = ((N + 31) / 32) * 4;
  constexpr int pbase = kWaves == 8 ? 256 : 0;
  constexpr int NT = 64 * kWaves, XT = kWaves == 8 ? 256 : NT, PTH = NT - pbase;
  constexpr int RX = ((QM / 8) * (2 * PT) + XT - 1) / XT;    // kch * pch <= QM/8 * TN/8
  constexpr int RP = (2 * (NM / 8) * (2 * PT) + PTH - 1) / PTH;
  constexpr int RQ = (QM + NT - 1) / NT;
  constexpr int ROUNDS = RX > RP ? (RX > RQ ? RX : RQ) : (RP > RQ ? RP : RQ);
  static_assert(QM != kQmax || NM != kNmax || ROUNDS == 1, "the default build stages in one round");
  auto stage = [&](int rd) {
    const int xi = tid + rd * XT, tp = tid - pbase + rd * PTH, qi = tid + rd * NT;
    const bool do_x = (ROUNDS == 1 || tid < XT) && xi < kch * pch;
    const bool do_p = tp >= rd * PTH && tp < 2 * nch * pch;
    const int x_kc = xi % kch, x_pc = xi / kch;
    const int p_h = tp & 1, p_nc = (tp >> 1) % nch, p_pc = (tp >> 1) / nch;
    u32x4_t xr[8];
    f32x4_t pr[8];
    float dA_v = 0.f, dt_v = 0.f, dA_e = 0.f;
    if (qi < Q) {
      dA_v = side_at<F16>(p.dA, sidx + qi);
      dt_v = side_at<F16>(p.dt, sidx + qi);
      dA_e = side_at<F16>(p.dA, sidx + min(qi | 31, Q - 1));  // last key of qi's 32-key block
    }
    if (do_x) {
      const int pg = p0 + x_pc * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = x_kc * 8 + e;
        xr[e] = (k < Q && pg < P) ? *reinterpret_cast<const u32x4_t*>(xg + (int64_t)k * P + pg)
                                  : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    if (do_p) {
      const int pg = p0 + p_pc * 8 + 4 * p_h;   // P % 8 == 0: pg < P covers pg + 3
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int n = p_nc * 8 + e;
        if (n < N && pg < P) {
          if constexpr (F16) {
            const u32x2_t w = *reinterpret_cast<const u32x2_t*>(pvh + (int64_t)n * P + pg);
            pr[e] = f32x4_t{lo16<true>(w[0]), hi16<true>(w[0]), lo16<true>(w[1]), hi16<true>(w[1])};
          } else {
            pr[e] = *reinterpret_cast<const f32x4_t*>(pvg + (int64_t)n * P + pg);
          }
        } else {
          pr[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    if (qi < Q) {
      constexpr float kLog2e = 1.4426950408889634f;
      s_dA[qi] = dA_v * kLog2e;  // log2 domain
      s_dt[qi] = dt_v;
      // U[k] = exp2(dA[k_e] - dA[k]) dt[k], k_e = last key of k's 32-key block:
      // the k-dependent factor of W on blocks that lie wholly below a row
      s_U[qi] = fast_exp2((dA_e - dA_v) * kLog2e) * dt_v;
    }
    if (do_x) {
      u32x4_t tr[8];
      transpose8x8(xr, tr);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int row = x_pc * 8 + u;
        xT[row * XROW + (x_kc ^ (row & 15))] = tr[u];
      }
    }
    if (do_p) {
      // prevT split into bf16 hi + lo (the state term keeps ~16 mantissa bits),
      // packed straight into the transposed layout: dword j of pT row p holds
      // n = 8 p_nc + 2j, 2j + 1.  An f16 prevT is exact in f16, so its lo half
      // is zero and never used.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pp = p_pc * 8 + 4 * p_h + i;
        u32x4_t hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = pr[2 * j][i], c = pr[2 * j + 1][i];
          const uint32_t hw = pack2<F16>(a, c);
          hi[j] = hw;
          lo[j] = pack2<F16>(a - lo16<F16>(hw), c - hi16<F16>(hw));
        }
        pT[0][pp * PROW + (p_nc ^ (pp & 15))] = hi;
        if constexpr (!F16) pT[1][pp * PROW + (p_nc ^ (pp & 15))] = lo;
      }
    }
  };
  stage(0);
  for (int rd = 1; rd < ROUNDS; ++rd) stage(rd);
  __syncthreads();

#pragma unroll
  for (int ti = 0; ti < MAXT; ++ti) {
    if (tile_of(ti) >= nmt16) continue;
    if constexpr (!kCbAhead) fetch_cb(ti, bbuf[0]);
    if (ti + 1 < MAXT) {
      fetch_c(ti + 1, cbuf[(ti + 1) & 1]);
      if constexpr (kCbAhead) fetch_cb(ti + 1, bbuf[(ti + 1) & 1]);
    }
    const u32x4_t(&rc)[NSN] = cbuf[ti & 1].c;
    const u32x4_t(&rcb)[NKS] = bbuf[kCbAhead ? (ti & 1) : 0].cb;
    const int mrow0 = m0 + 16 * tile_of(ti);
    const int am = mrow0 + rr;  // this lane's output row
    // state and intra-chunk terms accumulate separately and meet only at the
    // store, so no VALU touches an accumulator between MFMAs
    f32x4_t acc_s[PT], acc[PT];
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) {
      acc_s[pt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc[pt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    // ---- state term: C[m, :] . prevT[:, p] (hi + lo), then * exp(dA[m])
#pragma unroll
    for (int ns = 0; ns < NSN; ++ns) {
      if (ns * 32 >= N) continue;  // pT is staged (zero-padded) only up to N rounded to 32
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        const int pp = pt * 16 + rr;
        const int ch = (ns * 4 + g4) ^ (pp & 15);
        acc_s[pt] = mfma16t<F16>(pT[0][pp * PROW + ch], rc[ns], acc_s[pt]);
        if constexpr (!F16) acc_s[pt] = mfma16t<F16>(pT[1][pp * PROW + ch], rc[ns], acc_s[pt]);
      }
    }
    const float dAm = am < Q ? s_dA[am] : 0.f;
    const float em = am < Q ? fast_exp2(dAm) : 0.f;

    // ---- intra-chunk term: W[m, k] . x[k, p] for k <= m, with the skip
    // connection folded into the diagonal: W[m, m] += D[h].  A 32-key block
    // that ends below the tile's first row uses the factored form
    //   W = cb[m, k] * U[k] * exp2(dA[m] - dA[k_e])   (both exponents <= 0);
    // the block(s) reaching the diagonal use exp2(dA[m] - dA[k]) per element,
    // masked to k <= m.
    const int kend = min(mrow0 + 16, Q);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks * 32 >= kend) continue;
      const int kb = ks * 32 + g4 * 8;
      float wv[8];
      if (ks * 32 + 31 < mrow0) {
        const f32x4_t u0 = *reinterpret_cast<const f32x4_t*>(s_U + kb);
        const f32x4_t u1 = *reinterpret_cast<const f32x4_t*>(s_U + kb + 4);
        const float vm = fast_exp2(dAm - s_dA[ks * 32 + 31]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t word = rcb[ks][e >> 1];
          const float cbf = (e & 1) ? hi16<F16>(word) : lo16<F16>(word);
          wv[e] = cbf * (e < 4 ? u0[e] : u1[e - 4]) * vm;
        }
      } else {
        const f32x4_t dA0 = *reinterpret_cast<const f32x4_t*>(s_dA + kb);
        const f32x4_t dA1 = *reinterpret_cast<const f32x4_t*>(s_dA + kb + 4);
        const f32x4_t dt0 = *reinterpret_cast<const f32x4_t*>(s_dt + kb);
        const f32x4_t dt1 = *reinterpret_cast<const f32x4_t*>(s_dt + kb + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = kb + e;
          const uint32_t word = rcb[ks][e >> 1];
          const float cbf = (e & 1) ? hi16<F16>(word) : lo16<F16>(word);
          const float dAk = e < 4 ? dA0[e] : dA1[e - 4];
          const float dtk = e < 4 ? dt0[e] : dt1[e - 4];
          float w = (k <= am && k < Q) ? cbf * fast_exp2(dAm - dAk) * dtk : 0.f;
          if (k == am) w += Dh;
          wv[e] = w;
        }
      }
      u32x4_t ahi, alo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t hw = pack2<F16>(wv[2 * i], wv[2 * i + 1]);
        ahi[i] = hw;
        alo[i] = pack2<F16>(wv[2 * i] - lo16<F16>(hw), wv[2 * i + 1] - hi16<F16>(hw));
      }
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        const int pp = pt * 16 + rr;
        const u32x4_t xb = xT[pp * XROW + ((ks * 4 + g4) ^ (pp & 15))];
        acc[pt] = mfma16t<F16>(xb, ahi, acc[pt]);
        acc[pt] = mfma16t<F16>(xb, alo, acc[pt]);
      }
    }

    // ---- store.  A full 16-row tile of 64 columns goes out as whole
    // 128-byte rows: each half (8 rows) is staged in this wave's 1 KB of LDS
    // and stored 16 bytes per lane (the register layout gives each lane 8
    // bytes of 16 rows per store, partial lines).  The row's 32-byte groups
    // are XOR-swizzled by row bits 1-2, so one column group's staging write
    // (32 bytes from each of the 8 rows) covers all 64 banks once.
    // Otherwise four consecutive columns per lane.
    if constexpr (PT == 4) {
      if (mrow0 + 16 <= mend && p0 + 64 <= P) {
        char* const st = reinterpret_cast<char*>(ostage + wave * 64);
        const int sr = rr & 7;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if ((rr >> 3) == h) {
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
              const f32x4_t o = acc_s[pt] * em + acc[pt];
              *reinterpret_cast<u32x2_t*>(st + sr * 128 + ((pt ^ ((sr >> 1) & 3)) * 32) + g4 * 8) =
                  u32x2_t{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
            }
          }
          lds_order();
          const int lr8 = lane >> 3, c = lane & 7;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
              st + lr8 * 128 + (((c >> 1) ^ ((lr8 >> 1) & 3)) * 32) + (c & 1) * 16);
          lds_order();
          *reinterpret_cast<u32x4_t*>(og + (int64_t)(mrow0 + 8 * h + lr8) * P + p0 + c * 8) = v;
        }
        continue;
      }
    }
    if (am < mend) {
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        const int pg = p0 + pt * 16 + 4 * g4;
        const f32x4_t o = acc_s[pt] * em + acc[pt];
        if (pg < P)
          *reinterpret_cast<u32x2_t*>(og + (int64_t)am * P + pg) =
              u32x2_t{pack2<F16>(o[0], o[1]), pack2<F16>(o[2], o[3])};
      }
    }
  }
}

template <int PT, bool F16>
void launch_mamba(const MambaParams& p, hipStream_t st) {
  const int64_t nblocks = (int64_t)p.Bb * p.nc * p.H * p.nmt * p.npt;
  // chunks longer than 256 or states wider than 128: the long build, 4 waves
  if (p.Q > kQmax || p.N > kNmax)
    hipLaunchKernelGGL((mamba_chunk_scan_kernel<PT, F16, 4, kQbig, kNbig>), dim3((unsigned)nblocks),
                       dim3(256), 0, st, p);
  // 8 waves when the m-tile holds 8 or more 16-row tiles (tile_m >= 128)
  else if (p.tile_m >= 128)
    hipLaunchKernelGGL((mamba_chunk_scan_kernel<PT, F16, 8>), dim3((unsigned)nblocks), dim3(512), 0,
                       st, p);
  else
    hipLaunchKernelGGL((mamba_chunk_scan_kernel<PT, F16, 4>), dim3((unsigned)nblocks), dim3(256), 0,
                       st, p);
}

template <bool F16>
int chunk_scan_impl(
    const void* cb, const void* x, const void* dt, const void* dA_cumsum, const void* C,
    const void* D, const void* prev_states_T, void* out, int64_t batch, int64_t nchunks,
    int64_t nheads, int64_t ngroups, int64_t chunk_size, int64_t headdim, int64_t dstate,
    int64_t tile_b, int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, void* stream, char* err, size_t errlen) {
  const char* fn = "helion_mamba2_chunk_scan_kernel";
  if (!cb || !x || !dt || !dA_cumsum || !C || !D || !prev_states_T || !out)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: null tensor pointer", fn);
  if (batch <= 0 || nchunks <= 0 || nheads <= 0 || ngroups <= 0 || chunk_size <= 0 ||
      headdim <= 0 || dstate <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: extents must be positive", fn);
  if (nheads % ngroups != 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: nheads %% ngroups != 0", fn);
  // size-1 subviews in b, h and c with offsets iv*tile: any other tile skips
  // work in the reference (mlir :29-34,46,49,62), so it is rejected here
  if (tile_b != 1 || tile_h != 1 || tile_c != 1)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: tile_b, tile_h and tile_c must be 1", fn);
  if (tile_m <= 0 || tile_n <= 0 || tile_k <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: tile sizes must be positive", fn);
  // tile_m is bounded by chunk_size (the m rows of one chunk) and tile_n by
  // headdim (natural_ub); each runs on the smallest built tile covering it
  // (the largest built one above).  tile_k tiles the keys of a chunk and is
  // only validated: the kernel walks a chunk's keys in 32-key blocks whatever
  // it is, and its bound is the example's loom.sym upper_bound (8192,
  // examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:3), or
  // chunk_size where that is larger.
  static const int64_t kMTiles[4] = {64, 128, 192, 256};
  static const int64_t kNTiles[3] = {16, 32, 64};
  const int64_t wm = loom_fit_tile(tile_m, chunk_size, kMTiles, 4);
  const int64_t wn = loom_fit_tile(tile_n, headdim, kNTiles, 3);
  const int64_t k_ub = std::max<int64_t>(kMambaTileKBound, chunk_size);
  if (wm == 0 || wn == 0 || tile_k > k_ub)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "%s: tiles exceed their bounds (natural_ub): tile_m=%lld (chunk_size=%lld), "
                     "tile_n=%lld (headdim=%lld), tile_k=%lld (%lld)",
                     fn, (long long)tile_m, (long long)chunk_size, (long long)tile_n,
                     (long long)headdim, (long long)tile_k, (long long)k_ub);
  if (wm < 0 || wn < 0)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "%s: tile_m=%lld, tile_n=%lld: each must be a multiple of 16 (the MFMA tile "
                     "edge) or its whole extent",
                     fn, (long long)tile_m, (long long)tile_n);
  tile_m = wm;
  tile_n = wn;
  if (chunk_size > kQbig || dstate > kNbig || chunk_size % 8 || dstate % 8 || headdim % 8)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "%s: built for chunk_size <= %d, dstate <= %d, both and headdim multiples "
                     "of 8",
                     fn, kQbig, kNbig);
  if (!aligned16(cb) || !aligned16(x) || !aligned16(C) || !aligned16(prev_states_T) ||
      !aligned16(out))
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: tensors must be 16-byte aligned", fn);
  const int64_t nmt = cdiv64(chunk_size, tile_m), npt = cdiv64(headdim, tile_n);
  if (!loom_prod_le({batch, nchunks, nheads, nmt, npt}, 0x7fffffff) ||
      !loom_prod_le({batch, nheads, nchunks, chunk_size, headdim}, (int64_t)1 << 40) ||
      !loom_prod_le({batch, nchunks, nheads, dstate, headdim}, (int64_t)1 << 40) ||
      !loom_prod_le({batch, nchunks, ngroups, chunk_size, chunk_size}, (int64_t)1 << 40))
    return loom_fail(err, errlen, LOOM_EINVAL, "%s: problem too large", fn);
  MambaParams p{};
  p.cb = static_cast<const uint16_t*>(cb);
  p.x = static_cast<const uint16_t*>(x);
  p.dt = dt;
  p.dA = dA_cumsum;
  p.C = static_cast<const uint16_t*>(C);
  p.Dh = D;
  p.prevT = prev_states_T;
  p.out = static_cast<uint16_t*>(out);
  p.Bb = (int)batch;
  p.nc = (int)nchunks;
  p.H = (int)nheads;
  p.G = (int)ngroups;
  p.Q = (int)chunk_size;
  p.P = (int)headdim;
  p.N = (int)dstate;
  p.tile_m = (int)tile_m;
  p.tile_n = (int)tile_n;
  p.nmt = (int)nmt;
  p.npt = (int)npt;
  if (loom_validate_only()) return loom_ok(err, errlen);
  hipStream_t st = static_cast<hipStream_t>(stream);
  p.cus = stream_cus(st);
  if (tile_n == 64) launch_mamba<4, F16>(p, st);
  else if (tile_n == 32) launch_mamba<2, F16>(p, st);
  else launch_mamba<1, F16>(p, st);
  return loom_check_launch(err, errlen, fn);
}

}  // namespace

extern "C" {

int loom_hip_helion_mamba2_chunk_scan_kernel(
    const void* cb, const void* x, const void* dt, const void* dA_cumsum, const void* C,
    const void* D, const void* prev_states_T, void* out, int64_t batch, int64_t nchunks,
    int64_t nheads, int64_t ngroups, int64_t chunk_size, int64_t headdim, int64_t dstate,
    int64_t tile_b, int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, void* stream, char* err, size_t errlen) {
  return chunk_scan_impl<false>(cb, x, dt, dA_cumsum, C, D, prev_states_T, out, batch, nchunks,
                                nheads, ngroups, chunk_size, headdim, dstate, tile_b, tile_h,
                                tile_c, tile_m, tile_n, tile_k, stream, err, errlen);
}
int loom_hip_helion_mamba2_chunk_scan_kernel_f16(
    const void* cb, const void* x, const void* dt, const void* dA_cumsum, const void* C,
    const void* D, const void* prev_states_T, void* out, int64_t batch, int64_t nchunks,
    int64_t nheads, int64_t ngroups, int64_t chunk_size, int64_t headdim, int64_t dstate,
    int64_t tile_b, int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, void* stream, char* err, size_t errlen) {
  return chunk_scan_impl<true>(cb, x, dt, dA_cumsum, C, D, prev_states_T, out, batch, nchunks,
                               nheads, ngroups, chunk_size, headdim, dstate, tile_b, tile_h,
                               tile_c, tile_m, tile_n, tile_k, stream, err, errlen);
}

}  // extern "C"
