// attention.hip -- @attention (flash-attention forward) on gfx950.
//
// Reference: examples/flashattn/IR/00_from_helion_frontend.mlir:4-127.
//   k [BH, D, Skv] (keys transposed), v [BH, Skv, D], q [BH, Sq, D],
//   out [BH, Sq, D].  Per query row: m = -inf, l = 1, acc = 0 (:19-23); for
//   every KV tile: S = q.k (:38), m_ij = rowmax(S)*scale (:39-48),
//   m' = max(m, m_ij) (:49-54), P = exp(S*scale - m') (:55-70),
//   alpha = exp(m - m') (:77-86), l' = l*alpha + rowsum(P) (:87-96),
//   acc' = acc*alpha + P.V (:97-113); out = acc / l (:116-121).
//   `causal` (absent from the reference) makes key j visible to query i
//   only when j <= i; fully hidden KV blocks are skipped.
//   Any head dim that is a multiple of 8 up to 256 runs on the kernel built
//   for 64, 128 or 256: the K rows past it are copied from zeros, the Q
//   elements past it are zero, so the scores are exact; the V columns past it
//   only reach O columns that are never stored.
//
// gfx950 mapping (attention_dma_kernel below): a workgroup of W waves owns
// 16 QT W query rows of one (b, h) and streams K and V through LDS in
// 64-key blocks copied by LDS DMA; the MFMAs compute S^T = K^T Q^T and
// O^T += V^T P^T so P^T is built straight from the S^T accumulators.
// Softmax runs in fp32 in the log2 domain with a lazily moved base.  Causal
// tiles are launched heaviest first.
#include "common.h"

namespace {

struct AttnParams {
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* q;
  uint16_t* out;
  int BH, Sq, Skv, causal, nqt;
  int D;     // head dim: a multiple of 8, at most the kernel's D
  int koff32;  // D * Skv * 2 < 2^32: K's per-lane DMA offsets fit 32 bits
  float c2;  // scale * log2(e)
};

// ---------------------------------------------------------------------------
// LDS-DMA variant: K and V blocks are copied global -> LDS unchanged
// (global_load_lds_dwordx4, 3 stages of 64 keys, 2 at D 256), Ks [d][key] and
// Vs [key][d],
// and both operands that need k-contiguous data are built by
// ds_read_b64_tr_b16:
//   S^T[key, q]  = K^T . Q^T : row operand K^T from Ks (lane r gets key 16 jt + r,
//                              eight consecutive d) -- keys in natural order;
//   O^T[d, q]   += V^T . P^T : row operand V^T from Vs (lane r gets d = 16 dt + r,
//                              keys 16 j0 + 4 g + 0..3 and 16 j1 + 4 g + 0..3),
//                              exactly the keys P^T holds in lane group g.
// Four waves of 16 QT query rows share each K/V stage.  Softmax rescaling is
// lazy: a row's running max only moves (and O, l are rescaled) when a block
// raises it by more than 8 in the log2 domain, which keeps P <= 2^8 and the
// result exact (numerator and denominator share the stale base).
// Ks rows (128 B) and Vs rows (2 D bytes) XOR their 16-byte chunk index with
// k_swz / v_swz so that the 32 lanes of each pass of a transposed read touch
// distinct banks.  The banks repeat every 256 bytes (measured: rows 256 bytes
// apart conflict, SQ_LDS_BANK_CONFLICT), so a 32-byte row piece has eight
// positions per window.
// ---------------------------------------------------------------------------
// One pass of a K^T read covers Ks rows d..d+3 and d+8..d+11, 32 bytes each;
// 128-byte rows put the even rows on one half of the window and the odd rows
// on the other, so rows d, d^2, d^8, d^10 must take distinct chunk pairs:
// row bits 1 and 3 pick them (bit 0 only repeats the half's pattern).
LOOM_DEV int k_swz(int d) { return (2 * (d & 3)) ^ (2 * ((d >> 3) & 1)); }
// One pass of a V^T read covers 8 consecutive Vs rows, 32 bytes each.  D 128
// and 256 (rows of a multiple of 256 bytes): all eight share a window
// position, row bits 0-2 pick the pair.  D 64 (128-byte rows): rows r, r^2,
// r^4, r^6 share one, bits 1-2.
template <int D>
LOOM_DEV int v_swz(int k) { return D >= 128 ? 2 * (k & 7) : 2 * ((k >> 1) & 3); }
// Q / O staging rows (2 D bytes): chunk c of row lr sits at position
// c ^ q_swz(lr), so the 16 rows of a 32-lane pass (16-byte reads of chunks
// c and c + 1, or 8-byte halves of one chunk) land on distinct banks: rows
// 256 bytes apart at D 128, 128 bytes apart at D 64 (there bits 0-2 of the
// row XOR bit 3, which tells rows 8 apart apart).
template <int D>
LOOM_DEV int q_swz(int lr) { return D >= 128 ? (lr & 15) : ((lr ^ (lr >> 3)) & 7); }

// KREG (Skv not a multiple of 8): K rows [d][0..Skv) do not start on
// 16-byte boundaries, so K cannot be copied by 16-byte LDS DMA.  Each lane
// then loads its 16-byte pieces of a K block into registers (row_piece8: one
// 16-byte buffer load at any 2-byte aligned offset, 2-byte loads where a
// piece reaches past its row), issued before the block NS-1 stages ahead of
// the one being computed and written to the same LDS position after that
// computation; V keeps its DMA.
template <int D, int QT, int W, bool H, bool KREG>
__global__ void __launch_bounds__(64 * W) attention_dma_kernel(AttnParams p) {
  constexpr int KB = 64;                        // keys per stage
  // stages: three of 32 KB (K and V) up to D 128; two of 64 KB at D 256
  // (a fourth 32 KB stage measured 2% slower: causal B4 H32 S4096 572
  // against 561 us; two stages 554-557 us, equal within box noise)
  constexpr int NS = D > 128 ? 2 : 3;
  constexpr int BQ = 16 * QT * W;               // queries per workgroup
  constexpr int K_BYTES = D * KB * 2, V_BYTES = KB * D * 2;
  constexpr int K_INSTR = K_BYTES / 1024 / W;   // DMA instructions per wave per stage
  constexpr int V_INSTR = V_BYTES / 1024 / W;
  static_assert(K_INSTR >= 1 && V_INSTR >= 1, "every wave issues K and V copies");
  constexpr int LPW = K_INSTR + V_INSTR;
  constexpr int VROW = D * 2;                   // Vs row bytes
  constexpr int V_ROWS_PER_I = 1024 / VROW;
  constexpr int DSTEPS = D / 32, DT = D / 16;
  static_assert(LPW * (NS - 2) <= 63, "vmcnt range");
  // Q reaches LDS by DMA up to D 128 (a region after the stages, which also
  // stages O for the epilogue); at D 256 the two 64 KB stages leave no room
  // and Q is loaded into registers
  constexpr bool QDMA = D <= 128;
  constexpr int QROW = D * 2;                   // Q / O staging row bytes
  constexpr int Q_LDS = QDMA ? BQ * QROW : 0;
  constexpr int Q_INSTR = QDMA ? Q_LDS / 1024 / W : 0;   // Q copies per wave
  static_assert(!QDMA || Q_LDS % (1024 * W) == 0, "whole Q copies per wave");
  constexpr int STAGE = K_BYTES + V_BYTES;
  static_assert(NS * STAGE + Q_LDS <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[NS * STAGE + Q_LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int a4 = r >> 2, c4 = r & 3;            // transposed-read lane roles

  const int L = blockIdx.x;
  const int qtile = p.nqt - 1 - L / p.BH;       // heaviest tiles first
  const int bh = L % p.BH;
  const int q0 = qtile * BQ;
  const int Sq = p.Sq, Skv = p.Skv, Dr = p.D;
  const uint16_t* __restrict__ kg = p.k + (int64_t)bh * Dr * Skv;
  const uint16_t* __restrict__ vg = p.v + (int64_t)bh * Skv * Dr;
  const uint16_t* __restrict__ qg = p.q + (int64_t)bh * Sq * Dr;

  auto stK = [&](int s) -> lds_char_t* { return (lds_char_t*)(smem + s * STAGE); };
  auto stV = [&](int s) -> lds_char_t* { return (lds_char_t*)(smem + s * STAGE + K_BYTES); };
  lds_char_t* const sQ = (lds_char_t*)(smem + NS * STAGE);
  // ---- DMA of block `blk` into stage s (keys past Skv are clamped: masked
  // later; Ks rows d >= Dr, eight to a copy, come from zeros; Vs chunks past
  // Dr repeat the row's last chunk).  A whole block inside [0, Skv) takes
  // each copy as the block's scalar base plus this lane's byte offset, both
  // computed once (no VALU per copy); the last, partial block clamps every
  // lane's key (and K offsets past 32 bits always do).
  uint32_t koff[K_INSTR], voff[V_INSTR];
#pragma unroll
  for (int i = 0; i < K_INSTR; ++i) {
    const int j = wave * K_INSTR + i, d = j * 8 + lane / 8;
    // unsigned: it wraps (and goes unused, koff32 == 0) when D * Skv * 2 >= 2^32
    koff[i] = ((uint32_t)d * (uint32_t)Skv + (uint32_t)(((lane % 8) ^ k_swz(d)) * 8)) * 2u;
  }
#pragma unroll
  for (int i = 0; i < V_INSTR; ++i) {
    const int j = wave * V_INSTR + i, kr = j * V_ROWS_PER_I + lane / (D / 8);
    voff[i] = (uint32_t)(kr * Dr + min((lane % (D / 8)) ^ v_swz<D>(kr), Dr / 8 - 1) * 8) * 2;
  }
  auto issue = [&](int s, int blk) {
    const int kv0 = blk * KB;
    const uint32_t lk = lds_addr(stK(s)), lv = lds_addr(stV(s));
    if (kv0 + KB <= Skv && (KREG || p.koff32)) {               // wave-uniform
      if constexpr (!KREG) {
#pragma unroll
        for (int i = 0; i < K_INSTR; ++i) {
          const int j = wave * K_INSTR + i;
          if (j * 8 < Dr)
            dma_load16_s(koff[i], kg + kv0, lk + j * 1024);
          else
            dma_load16(loom_zero_kb + lane * 4, lk + j * 1024);
        }
      }
#pragma unroll
      for (int i = 0; i < V_INSTR; ++i)
        dma_load16_s(voff[i], vg + (int64_t)kv0 * Dr, lv + (wave * V_INSTR + i) * 1024);
      return;
    }
    if constexpr (!KREG) {
#pragma unroll
      for (int i = 0; i < K_INSTR; ++i) {
        const int j = wave * K_INSTR + i;
        const int d = j * 8 + lane / 8;                     // Ks row
        const int c = (lane % 8) ^ k_swz(d);
        const int key = min(kv0 + c * 8, Skv - 8);
        if (j * 8 < Dr)                                     // wave-uniform
          dma_load16(kg + (int64_t)d * Skv + key, lk + j * 1024);
        else
          dma_load16(loom_zero_kb + lane * 4, lk + j * 1024);
      }
    }
#pragma unroll
    for (int i = 0; i < V_INSTR; ++i) {
      const int j = wave * V_INSTR + i;
      const int kr = j * V_ROWS_PER_I + lane / (D / 8);   // Vs row (key)
      const int c = min((lane % (D / 8)) ^ v_swz<D>(kr), Dr / 8 - 1);
      const int key = min(kv0 + kr, Skv - 1);
      dma_load16(vg + (int64_t)key * Dr + c * 8, lv + j * 1024);
    }
  };

  // ---- KREG: this lane's K pieces of block `blk` (the DMA's positions:
  // row d, 8 keys from kv0 + 8 c) into registers (row_piece8), then into
  // stage s; k needs only 2-byte alignment
  const rsrc_t krs = make_rsrc(kg, KREG ? (uint32_t)(Dr * Skv * 2) : 0u);
  u32x4_t kr[KREG ? K_INSTR : 1];
  auto kload = [&](int blk) {
    const int kv0 = blk * KB;
#pragma unroll
    for (int i = 0; i < K_INSTR; ++i) {
      const int j = wave * K_INSTR + i;
      const int d = j * 8 + lane / 8;
      const int c = (lane % 8) ^ k_swz(d);
      kr[i] = j * 8 < Dr ? row_piece8(krs, Skv, d, kv0 + c * 8)   // padding rows: zeros
                         : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto kstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < K_INSTR; ++i)
      *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(
          stK(s) + (wave * K_INSTR + i) * 1024 + lane * 16) = kr[i];
  };

  const int kv_end = p.causal ? min(Skv, q0 + BQ) : Skv;
  const int nblk = (kv_end + KB - 1) / KB;
  // ---- Q by LDS DMA (D <= 128): local query row lr of the workgroup at
  // sQ + lr QROW, its 16-byte chunk c at position c ^ q_swz(lr) (rows past Sq
  // repeat the last; chunks past Dr repeat the row's last one and are zeroed
  // when read).  Issued before the first K/V stages, so the hand-placed wait
  // for stage 0 covers Q too (copies complete in issue order): a register
  // load of Q would make the compiler wait for every copy issued before it.
  if constexpr (QDMA) {
    const uint32_t lq = lds_addr(sQ);
#pragma unroll
    for (int i = 0; i < Q_INSTR; ++i) {
      const int j = wave * Q_INSTR + i;
      const int e = j * 1024 + lane * 16;                  // byte of the Q region
      const int lr = e / QROW, cp = (e % QROW) / 16;
      const int c = min(cp ^ q_swz<D>(lr), Dr / 8 - 1);
      const int qrow = min(q0 + lr, Sq - 1);
      dma_load16(qg + (int64_t)qrow * Dr + c * 8, lq + j * 1024);
    }
  }
  // the first NS-1 KV blocks start loading before the loop (at D 256, before
  // Q too, so their latency and Q's overlap)
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nblk) {
      if constexpr (KREG) {
        kload(s);
        kstore(s);
      }
      issue(s, s);
    }

  // ---- Q^T operands: lane holds q[q0w + 16 qt + r][32 ds + 8 g .. +7] times
  // scale * log2(e), rounded to bf16, so scores come out in the log2 domain
  // (zero past Dr)
  const int q0w = q0 + 16 * QT * wave;
  u32x4_t qf[DSTEPS][QT];
  auto q_operand = [&](int qt, int ds, u32x4_t raw) {
    if (ds * 32 + g * 8 >= Dr) raw = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      qf[ds][qt][e] = pack2<H>(lo16<H>(raw[e]) * p.c2, hi16<H>(raw[e]) * p.c2);
  };
  if constexpr (!QDMA) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qrow = min(q0w + 16 * qt + r, Sq - 1);
#pragma unroll
      for (int ds = 0; ds < DSTEPS; ++ds) {
        const int d0 = min(ds * 32 + g * 8, Dr - 8);
        q_operand(qt, ds, *reinterpret_cast<const u32x4_t*>(qg + (int64_t)qrow * Dr + d0));
      }
    }
  }

  // running base m (log2 domain) per query row; O^T and the row sums l (an
  // MFMA of P^T against ones: every row of that tile holds l) share it
  // negm[qt] holds -m in all four lanes of a quad: the accumulator every
  // score tile starts from, kept across blocks and rebuilt only when m moves
  float m_run[QT];
  f32x4_t negm[QT];
  f32x4_t ot[DT][QT], lacc[QT];
  const u32x4_t ones = u32x4_t{kOnePair<H>, kOnePair<H>, kOnePair<H>, kOnePair<H>};
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = 0.f;
    negm[qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    lacc[qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) ot[dt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](int s, int blk) {
    const int kv0 = blk * KB;
    // a wave whose queries all precede the block sees only masked keys
    if (p.causal && kv0 > q0w + 16 * QT - 1) return;
    const lds_char_t* ks = stK(s);
    const lds_char_t* vs = stV(s);
    const bool edge = kv0 + KB > Skv || (p.causal && kv0 + KB - 1 > q0w);
    // two 32-key halves, each a softmax step of its own
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // ---- S^T = K^T Q^T - m; st[j][qt][i] = score of key kv0 + 32 h + 16 j + 4 g + i
      f32x4_t st[2][QT];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) st[j][qt] = negm[qt];
#pragma unroll
      for (int ds = 0; ds < DSTEPS; ++ds) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int jt = 2 * h + j;
          const int d = ds * 32 + g * 8 + a4;               // & 3 == a4
          const int ch = (2 * jt + (c4 >> 1)) ^ k_swz(d);
          const lds_char_t* q = ks + d * (KB * 2) + ch * 16 + (c4 & 1) * 8;
          const u32x2_t lo = lds_read_tr16(q);
          const u32x2_t hi = lds_read_tr16(q + 4 * (KB * 2));
          const u32x4_t kf = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) st[j][qt] = mfma16t<H>(kf, qf[ds][qt], st[j][qt]);
        }
      }
      // ---- masking (only blocks that reach past Skv or the diagonal)
      if (edge) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int qrow = q0w + 16 * qt + r;
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kv0 + 32 * h + 16 * j + 4 * g + i;
              if (key >= Skv || (p.causal && key > qrow)) st[j][qt][i] = -INFINITY;
            }
        }
      }
      // ---- lazy online softmax.  P = 2^(s - m) directly while every score
      // stays within 2^8 of the base; the first step, or a step that rises
      // higher, moves m to the row maximum and rescales O and l (numerator
      // and denominator share m, so the result does not depend on it)
      float lmax[QT];
      bool big = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[j][qt][i]);
        lmax[qt] = mx;
        big |= mx > 8.f;
      }
      const bool first = blk == 0 && h == 0;
      if (first || __builtin_amdgcn_ballot_w64(big) != 0) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float mx = lmax[qt];
          mx = fmaxf(mx, __shfl_xor(mx, 16));
          mx = fmaxf(mx, __shfl_xor(mx, 32));
          // the first step sets m (O and l are still zero); later ones only raise it
          const float shift = first ? (mx == -INFINITY ? 0.f : mx) : fmaxf(mx, 0.f);
          if (!first) {
            const float alpha = fast_exp2(-shift);
            lacc[qt] *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) ot[dt][qt] *= alpha;
          }
          m_run[qt] += shift;
          negm[qt] = f32x4_t{-m_run[qt], -m_run[qt], -m_run[qt], -m_run[qt]};
#pragma unroll
          for (int j = 0; j < 2; ++j) st[j][qt] -= shift;
        }
      }
      // ---- O^T += V^T P^T and l += ones . P^T over these 32 keys
      u32x4_t pf[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        f32x4_t e0, e1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e0[i] = fast_exp2(st[0][qt][i]);
          e1[i] = fast_exp2(st[1][qt][i]);
        }
        pf[qt] = u32x4_t{pack2<H>(e0[0], e0[1]), pack2<H>(e0[2], e0[3]),
                         pack2<H>(e1[0], e1[1]), pack2<H>(e1[2], e1[3])};
        lacc[qt] = mfma16t<H>(ones, pf[qt], lacc[qt]);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int k0r = 32 * h + 4 * g + a4;
        const int ch = (2 * dt + (c4 >> 1)) ^ v_swz<D>(k0r);
        const lds_char_t* q = vs + k0r * VROW + ch * 16 + (c4 & 1) * 8;
        const u32x2_t lo = lds_read_tr16(q);                // keys 32h + 4g + 0..3
        const u32x2_t hi = lds_read_tr16(q + 16 * VROW);    // keys 32h + 16 + 4g + 0..3
        const u32x4_t vf = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) ot[dt][qt] = mfma16t<H>(vf, pf[qt], ot[dt][qt]);
      }
    }
  };

  // ---- pipeline: NS stages (the first NS-1 issued above), waits placed by
  // hand as in gemm.hip
  for (int it0 = 0; it0 < nblk; it0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int it = it0 + s;
      if (it < nblk) {
        const int younger = min(NS - 2, nblk - 1 - it);
        if (younger >= 2) LOOM_WAIT_VMCNT(2 * LPW);
        else if (younger == 1) LOOM_WAIT_VMCNT(LPW);
        else LOOM_WAIT_VMCNT(0);
        // KREG: this wave's K stores of the previous iteration are in LDS
        if constexpr (KREG) LOOM_WAIT_LGKM0();
        barrier_nofence();
        if constexpr (QDMA) {
          if (it == 0) {
            // this wave's Q^T operands from the Q region (landed with stage 0)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
              const int lr = 16 * QT * wave + 16 * qt + r;
#pragma unroll
              for (int ds = 0; ds < DSTEPS; ++ds)
                q_operand(qt, ds, *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                                      sQ + lr * QROW + ((4 * ds + g) ^ q_swz<D>(lr)) * 16));
            }
          }
        }
        const bool ahead = it + NS - 1 < nblk;
        if constexpr (KREG) {
          if (ahead) kload(it + NS - 1);
        }
        if (ahead) issue((s + NS - 1) % NS, it + NS - 1);
        compute(s, it);
        // KREG: the stage written here was last read before this
        // iteration's barrier (block it - 1); the compiler waits for the
        // loads (and, since it cannot tell them apart, everything older)
        if constexpr (KREG) {
          if (ahead) kstore((s + NS - 1) % NS);
        }
      }
    }
  }

  // ---- out = acc / l; ot[dt][qt][i] is d = 16 dt + 4 g + i of query q0w + 16 qt + r.
  // With D <= 128 and rows of exactly D, each wave stages its rows in its
  // own slice of the Q region (nothing else touches it after the first
  // block) and writes them back as whole rows, 16 bytes per lane: 8-byte
  // stores of 32-byte row pieces cost the workgroup's end far more.
  if constexpr (QDMA) {
    if (Dr == D) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const float inv = 1.f / lacc[qt][0];
        const int lr = 16 * QT * wave + 16 * qt + r;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const f32x4_t o = ot[dt][qt];
          const int pos = (2 * dt + (g >> 1)) ^ q_swz<D>(lr);
          *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(
              sQ + lr * QROW + pos * 16 + (g & 1) * 8) =
              u32x2_t{pack2<H>(o[0] * inv, o[1] * inv), pack2<H>(o[2] * inv, o[3] * inv)};
        }
      }
      constexpr int CPR = QROW / 16;                      // chunks per row
      lds_order();
#pragma unroll
      for (int k = 0; k < 16 * QT * CPR / 64; ++k) {
        const int idx = k * 64 + lane;
        const int lr = 16 * QT * wave + idx / CPR, cp = idx % CPR;
        const u32x4_t v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
            sQ + lr * QROW + cp * 16);
        if (q0 + lr < Sq)
          *reinterpret_cast<u32x4_t*>(p.out + ((int64_t)bh * Sq + q0 + lr) * Dr +
                                      (cp ^ q_swz<D>(lr)) * 8) = v;
      }
      return;
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    __builtin_amdgcn_sched_barrier(0);
    const float inv = 1.f / lacc[qt][0];
    const int qrow = q0w + 16 * qt + r;
    if (qrow < Sq) {
      uint16_t* orow = p.out + ((int64_t)bh * Sq + qrow) * Dr;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4_t o = ot[dt][qt];
        if (dt * 16 + 4 * g < Dr)
          *reinterpret_cast<u32x2_t*>(orow + dt * 16 + 4 * g) =
              u32x2_t{pack2<H>(o[0] * inv, o[1] * inv), pack2<H>(o[2] * inv, o[3] * inv)};
      }
    }
  }
}

template <bool H, bool KREG>
void launch_attention(const AttnParams& p, int64_t D, int64_t tile_m, hipStream_t st) {
  const dim3 grid((unsigned)(p.BH * p.nqt)), b4(256), b8(512);
  if (D == 256) {   // one 16-row query tile per wave: 64 or 128 queries
    if (tile_m == 64) hipLaunchKernelGGL((attention_dma_kernel<256, 1, 4, H, KREG>), grid, b4, 0, st, p);
    else hipLaunchKernelGGL((attention_dma_kernel<256, 1, 8, H, KREG>), grid, b8, 0, st, p);
    return;
  }
  switch ((D == 128 ? 10 : 0) + (int)(tile_m / 64)) {
    case 11: hipLaunchKernelGGL((attention_dma_kernel<128, 1, 4, H, KREG>), grid, b4, 0, st, p); break;
    case 12: hipLaunchKernelGGL((attention_dma_kernel<128, 1, 8, H, KREG>), grid, b8, 0, st, p); break;
    case 13: hipLaunchKernelGGL((attention_dma_kernel<128, 3, 4, H, KREG>), grid, b4, 0, st, p); break;
    case 14: hipLaunchKernelGGL((attention_dma_kernel<128, 2, 8, H, KREG>), grid, b8, 0, st, p); break;
    case 1: hipLaunchKernelGGL((attention_dma_kernel<64, 1, 4, H, KREG>), grid, b4, 0, st, p); break;
    case 2: hipLaunchKernelGGL((attention_dma_kernel<64, 1, 8, H, KREG>), grid, b8, 0, st, p); break;
    case 3: hipLaunchKernelGGL((attention_dma_kernel<64, 3, 4, H, KREG>), grid, b4, 0, st, p); break;
    default: hipLaunchKernelGGL((attention_dma_kernel<64, 2, 8, H, KREG>), grid, b8, 0, st, p); break;
  }
}

template <bool H>
int attention_impl(const void* k, const void* v, const void* q, void* out, int64_t BH,
                       int64_t Sq, int64_t Skv, int64_t D, float scale, int causal,
                       int64_t tile_b, int64_t tile_m, int64_t tile_n, void* stream, char* err,
                       size_t errlen) {
  if (!k || !v || !q || !out)
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: null tensor pointer");
  if (BH <= 0 || Sq <= 0 || Skv <= 0 || D <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: extents must be positive");
  if (tile_b <= 0 || tile_b > BH || tile_m <= 0 || tile_n <= 0 || tile_n > Skv)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "attention: tiles must satisfy 1 <= tile_b <= BH, 1 <= tile_n <= Skv "
                     "(tile_b=%lld tile_m=%lld tile_n=%lld)",
                     (long long)tile_b, (long long)tile_m, (long long)tile_n);
  if (causal && Sq != Skv)
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: causal needs Sq == Skv");
  // tile_m is bounded by Sq (natural_ub) and runs on the smallest built
  // query tile covering it (the largest above them: 256, or 128 for head dims
  // above 128); a query row's result does not depend on the workgroup that
  // holds it
  static const int64_t kQTiles[4] = {64, 128, 192, 256};
  const int64_t wm = loom_fit_tile(tile_m, Sq, kQTiles, D > 128 ? 2 : 4);
  if (wm == 0)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "attention: tile_m=%lld exceeds its extent Sq=%lld (natural_ub)",
                     (long long)tile_m, (long long)Sq);
  if (wm < 0)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "attention: tile_m=%lld must be a multiple of 16 (the MFMA tile edge) or Sq "
                     "itself",
                     (long long)tile_m);
  tile_m = wm;
  if (D % 8 != 0 || D > 256)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "attention: head_dim %lld not built (a multiple of 8 up to 256)",
                     (long long)D);
  // Skv not a multiple of 8 takes the register-staged K path (KREG), whose
  // K buffer descriptor addresses one (b, h)'s D x Skv keys in 32 bits
  const bool kreg = Skv % 8 != 0;
  if (kreg && !loom_prod_le({D, Skv, 2}, 0x7fffffffll))
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: D*Skv too large");
  if ((!kreg && !aligned16(k)) || (reinterpret_cast<uintptr_t>(k) & 1u) || !aligned16(v) ||
      !aligned16(q) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "attention: v and q must be 16-byte aligned, out 8-byte, k 16-byte (2-byte "
                     "when Skv is not a multiple of 8)");
  if (Sq > (1 << 30) || Skv > (1 << 30) || !loom_prod_le({BH, cdiv64(Sq, tile_m)}, 0x7fffffff) ||
      !loom_prod_le({BH, Sq, D}, (int64_t)1 << 50) || !loom_prod_le({BH, Skv, D}, (int64_t)1 << 50))
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: problem too large");
  AttnParams p{};
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q = static_cast<const uint16_t*>(q);
  p.out = static_cast<uint16_t*>(out);
  p.BH = (int)BH;
  p.Sq = (int)Sq;
  p.Skv = (int)Skv;
  p.causal = causal ? 1 : 0;
  p.nqt = (int)cdiv64(Sq, tile_m);
  p.D = (int)D;
  p.koff32 = loom_prod_le({D, Skv, 2}, 0xffffffffll) ? 1 : 0;
  p.c2 = scale * 1.4426950408889634f;
  if (loom_validate_only()) return loom_ok(err, errlen);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the kernel built for 64, 128 or 256 (the next one up) runs any narrower D
  const int64_t Dk = D <= 64 ? 64 : D <= 128 ? 128 : 256;
  if (kreg) launch_attention<H, true>(p, Dk, tile_m, st);
  else launch_attention<H, false>(p, Dk, tile_m, st);
  return loom_check_launch(err, errlen, "attention");
}

}  // namespace

extern "C" {

int loom_hip_attention(const void* k, const void* v, const void* q, void* out, int64_t BH,
                       int64_t Sq, int64_t Skv, int64_t D, float scale, int causal,
                       int64_t tile_b, int64_t tile_m, int64_t tile_n, void* stream, char* err,
                       size_t errlen) {
  return attention_impl<false>(k, v, q, out, BH, Sq, Skv, D, scale, causal, tile_b, tile_m,
                               tile_n, stream, err, errlen);
}
int loom_hip_attention_f16(const void* k, const void* v, const void* q, void* out, int64_t BH,
                           int64_t Sq, int64_t Skv, int64_t D, float scale, int causal,
                           int64_t tile_b, int64_t tile_m, int64_t tile_n, void* stream,
                           char* err, size_t errlen) {
  return attention_impl<true>(k, v, q, out, BH, Sq, Skv, D, scale, causal, tile_b, tile_m,
                              tile_n, stream, err, errlen);
}

}  // extern "C"
