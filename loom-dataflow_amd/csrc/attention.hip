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
//
// gfx950 mapping.  A workgroup owns tile_m query rows of one (b, h) and
// loops over 64-key blocks.  Each block of K and V is copied to LDS by
// register-transposed 8x8 blocks so both products read 16-byte operands:
//   Ks [key][d]  (K^T)  -- S^T[key, query] = K . Q^T, A operand from Ks,
//                          B operand Q^T kept in registers;
//   Vt [d][key]  (V^T)  -- O^T[d, query] += V^T . P^T, A operand from Vt,
//                          B operand P^T taken directly from the S^T
//                          accumulators (no shuffle, no LDS round trip).
// Inside a 32-key pair of S^T tiles the MFMA row -> key assignment is
// permuted (row rr of tile 2p+h holds key 32p + 8*(rr/4) + 4h + rr%4) so
// that every lane's eight P^T values are eight consecutive keys, matching
// one 16-byte read of Vt.  Softmax runs in fp32 in the log2 domain; rows'
// sums stay per lane until the end.  LDS rows are XOR-swizzled in 16-byte
// chunks so operand reads and transposed stores avoid bank conflicts.
// Causal tiles are launched heaviest first.
#include "common.h"

namespace {

constexpr int kKB = 64;       // keys per block
constexpr int kWaves = 4;

struct AttnParams {
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* q;
  uint16_t* out;
  int BH, Sq, Skv, causal, nqt;
  float c2;  // scale * log2(e)
};

// K^T row swizzle: distinct for the 8 keys {0..3, 8..11} (+4) read together
LOOM_DEV int kswz(int key) { return (key & 3) | (((key >> 3) & 1) << 2); }

template <int D, int QT>
__global__ void __launch_bounds__(64 * kWaves) attention_kernel(AttnParams p) {
  constexpr int BQ = 16 * QT * kWaves;     // queries per workgroup
  constexpr int DCH = D / 8;               // 16-byte chunks per Ks row
  constexpr int KCH = kKB / 8;             // 16-byte chunks per Vt row
  constexpr int DSTEPS = D / 32;
  constexpr int DT = D / 16;               // O^T tiles over d
  constexpr int NBLK = KCH * DCH;          // 8x8 blocks per K (and per V) tile
  static_assert(2 * NBLK <= 64 * kWaves, "one 8x8 block per copying thread");
  constexpr int KS_UNITS = kKB * DCH, VT_UNITS = D * KCH;
  constexpr int STAGE = KS_UNITS + VT_UNITS;
  __shared__ u32x4_t lds[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rr = lane & 15, g = lane >> 4;

  // heaviest (last) query tiles first; consecutive ids walk over (b, h)
  const int L = blockIdx.x;
  const int qtile = p.nqt - 1 - L / p.BH;
  const int bh = L % p.BH;
  const int q0 = qtile * BQ;
  const int Sq = p.Sq, Skv = p.Skv;

  const uint16_t* __restrict__ kg = p.k + (int64_t)bh * D * Skv;
  const uint16_t* __restrict__ vg = p.v + (int64_t)bh * Skv * D;
  const uint16_t* __restrict__ qg = p.q + (int64_t)bh * Sq * D;

  // ---- Q^T operand: lane holds q[qrow = q0 + 16*(QT*wave + qt) + rr][32 ds + 8 g ..]
  const int wq0 = q0 + 16 * QT * wave;
  u32x4_t qf[DSTEPS][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qrow = wq0 + 16 * qt + rr;
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds)
      qf[ds][qt] = qrow < Sq
                       ? *reinterpret_cast<const u32x4_t*>(qg + (int64_t)qrow * D + ds * 32 + g * 8)
                       : u32x4_t{0u, 0u, 0u, 0u};
  }

  // ---- copy roles: threads [0, NBLK) stage K blocks, [NBLK, 2 NBLK) V blocks
  const bool kcopy = tid < NBLK;
  const bool vcopy = !kcopy && tid < 2 * NBLK;
  const int ct = kcopy ? tid : tid - NBLK;
  // K: d-chunk fastest (conflict-free Ks stores); V: key-chunk fastest
  const int k_dc = ct % DCH, k_kc = ct / DCH;
  const int v_kc = ct % KCH, v_dc = ct / KCH;
  u32x4_t cr[8];

  auto load_block = [&](int kv0) {
    if (kcopy) {
      const int key = kv0 + k_kc * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        cr[e] = key < Skv ? *reinterpret_cast<const u32x4_t*>(kg + (int64_t)(k_dc * 8 + e) * Skv + key)
                          : u32x4_t{0u, 0u, 0u, 0u};
    } else if (vcopy) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = kv0 + v_kc * 8 + e;
        cr[e] = key < Skv ? *reinterpret_cast<const u32x4_t*>(vg + (int64_t)key * D + v_dc * 8)
                          : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  };
  auto store_block = [&](int stage) {
    u32x4_t tr[8];
    if (kcopy) {
      transpose8x8(cr, tr);  // tr[j] = d chunk k_dc of key 8 k_kc + j
      u32x4_t* ks = lds + stage * STAGE;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = k_kc * 8 + j;
        ks[key * DCH + (k_dc ^ kswz(key))] = tr[j];
      }
    } else if (vcopy) {
      transpose8x8(cr, tr);  // tr[u] = keys 8 v_kc .. +7 of d = 8 v_dc + u
      u32x4_t* vt = lds + stage * STAGE + KS_UNITS;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int d = v_dc * 8 + u;
        vt[d * KCH + (v_kc ^ (d & 7))] = tr[u];
      }
    }
  };

  float m_run[QT], l_run[QT];
  f32x4_t ot[DT][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) ot[dt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int kv_end = p.causal ? min(Skv, q0 + BQ) : Skv;
  const int nblk = (kv_end + kKB - 1) / kKB;
  if (nblk > 0) {
    load_block(0);
    store_block(0);
  }
  __syncthreads();

  for (int bi = 0; bi < nblk; ++bi) {
    const int kv0 = bi * kKB;
    if (bi + 1 < nblk) load_block(kv0 + kKB);
    const u32x4_t* ks = lds + (bi & 1) * STAGE;
    const u32x4_t* vt = ks + KS_UNITS;
    // a wave whose queries all precede the block sees only masked keys
    const bool active = !p.causal || kv0 <= wq0 + 16 * QT - 1;
    if (active) {
      // ---- S^T = K Q^T: tile jt = 2 pp + hh, row rr -> key 32pp + 8(rr/4) + 4hh + rr%4
      f32x4_t st[4][QT];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) st[jt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DSTEPS; ++ds) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          const int key = 32 * (jt >> 1) + 8 * (rr >> 2) + 4 * (jt & 1) + (rr & 3);
          const u32x4_t a = ks[key * DCH + ((ds * 4 + g) ^ kswz(key))];
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) st[jt][qt] = mfma16(a, qf[ds][qt], st[jt][qt]);
        }
      }
      // ---- online softmax; st[jt][qt][i] is key 32(jt/2) + 8g + 4(jt%2) + i
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int qrow = wq0 + 16 * qt + rr;
        float mx = -INFINITY;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kv0 + 32 * (jt >> 1) + 8 * g + 4 * (jt & 1) + i;
            float t = st[jt][qt][i] * p.c2;
            if (key >= Skv || (p.causal && key > qrow)) t = -INFINITY;
            st[jt][qt][i] = t;
            mx = fmaxf(mx, t);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run[qt], mx);
        // a row with no visible key so far keeps m = -inf; guard the exps
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_run[qt] - m_use);
        m_run[qt] = m_new;
        float ls = 0.f;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float pv = fast_exp2(st[jt][qt][i] - m_use);
            st[jt][qt][i] = pv;
            ls += pv;
          }
        l_run[qt] = l_run[qt] * alpha + ls;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) ot[dt][qt] *= alpha;
      }
      // ---- O^T += V^T P^T over the two 32-key pairs
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        u32x4_t pf[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          pf[qt] = u32x4_t{pack_bf16x2(st[2 * pp][qt][0], st[2 * pp][qt][1]),
                           pack_bf16x2(st[2 * pp][qt][2], st[2 * pp][qt][3]),
                           pack_bf16x2(st[2 * pp + 1][qt][0], st[2 * pp + 1][qt][1]),
                           pack_bf16x2(st[2 * pp + 1][qt][2], st[2 * pp + 1][qt][3])};
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = dt * 16 + rr;
          const u32x4_t a = vt[d * KCH + ((4 * pp + g) ^ (d & 7))];
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) ot[dt][qt] = mfma16(a, pf[qt], ot[dt][qt]);
        }
      }
    }
    if (bi + 1 < nblk) store_block((bi + 1) & 1);
    __syncthreads();
  }

  // ---- out = acc / l; O^T[dt][qt][i] is d = 16 dt + 4 g + i of query row
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float l = l_run[qt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.f / l;
    const int qrow = wq0 + 16 * qt + rr;
    if (qrow < Sq) {
      uint16_t* orow = p.out + ((int64_t)bh * Sq + qrow) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4_t o = ot[dt][qt];
        *reinterpret_cast<u32x2_t*>(orow + dt * 16 + 4 * g) =
            u32x2_t{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-DMA variant: K and V blocks are copied global -> LDS unchanged
// (global_load_lds_dwordx4, 4 stages of 64 keys), Ks [d][key] and Vs [key][d],
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
// 2 (row & 3), so a transposed read's four rows hit distinct banks.
// ---------------------------------------------------------------------------
template <int D, int QT>
__global__ void __launch_bounds__(256) attention_dma_kernel(AttnParams p) {
  constexpr int KB = 64;                        // keys per stage
  constexpr int NS = 4;                         // stages
  constexpr int BQ = 16 * QT * 4;               // queries per workgroup
  constexpr int K_BYTES = D * KB * 2, V_BYTES = KB * D * 2;
  constexpr int K_INSTR = K_BYTES / 1024 / 4;   // DMA instructions per wave per stage
  constexpr int V_INSTR = V_BYTES / 1024 / 4;
  constexpr int LPW = K_INSTR + V_INSTR;
  constexpr int VROW = D * 2;                   // Vs row bytes
  constexpr int V_ROWS_PER_I = 1024 / VROW;
  constexpr int DSTEPS = D / 32, DT = D / 16;
  static_assert(LPW * (NS - 2) <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char sK0[K_BYTES], sV0[V_BYTES];
  __shared__ __attribute__((aligned(1024))) char sK1[K_BYTES], sV1[V_BYTES];
  __shared__ __attribute__((aligned(1024))) char sK2[K_BYTES], sV2[V_BYTES];
  __shared__ __attribute__((aligned(1024))) char sK3[K_BYTES], sV3[V_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int a4 = r >> 2, c4 = r & 3;            // transposed-read lane roles

  const int L = blockIdx.x;
  const int qtile = p.nqt - 1 - L / p.BH;       // heaviest tiles first
  const int bh = L % p.BH;
  const int q0 = qtile * BQ;
  const int Sq = p.Sq, Skv = p.Skv;
  const uint16_t* __restrict__ kg = p.k + (int64_t)bh * D * Skv;
  const uint16_t* __restrict__ vg = p.v + (int64_t)bh * Skv * D;
  const uint16_t* __restrict__ qg = p.q + (int64_t)bh * Sq * D;

  auto stK = [&](int s) -> lds_char_t* {
    if (s == 0) return (lds_char_t*)sK0;
    if (s == 1) return (lds_char_t*)sK1;
    if (s == 2) return (lds_char_t*)sK2;
    return (lds_char_t*)sK3;
  };
  auto stV = [&](int s) -> lds_char_t* {
    if (s == 0) return (lds_char_t*)sV0;
    if (s == 1) return (lds_char_t*)sV1;
    if (s == 2) return (lds_char_t*)sV2;
    return (lds_char_t*)sV3;
  };
  // ---- DMA of block `blk` into stage s (keys past Skv are clamped: masked later)
  auto issue = [&](int s, int blk) {
    const int kv0 = blk * KB;
    const uint32_t lk = lds_addr(stK(s)), lv = lds_addr(stV(s));
#pragma unroll
    for (int i = 0; i < K_INSTR; ++i) {
      const int j = wave * K_INSTR + i;
      const int d = j * 8 + lane / 8;                     // Ks row
      const int c = (lane % 8) ^ (2 * (d & 3));
      const int key = min(kv0 + c * 8, Skv - 8);
      dma_load16(kg + (int64_t)d * Skv + key, lk + j * 1024);
    }
#pragma unroll
    for (int i = 0; i < V_INSTR; ++i) {
      const int j = wave * V_INSTR + i;
      const int kr = j * V_ROWS_PER_I + lane / (D / 8);   // Vs row (key)
      const int c = (lane % (D / 8)) ^ (2 * (kr & 3));
      const int key = min(kv0 + kr, Skv - 1);
      dma_load16(vg + (int64_t)key * D + c * 8, lv + j * 1024);
    }
  };

  // ---- Q^T operands: lane holds q[q0w + 16 qt + r][32 ds + 8 g .. +7]
  const int q0w = q0 + 16 * QT * wave;
  u32x4_t qf[DSTEPS][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qrow = min(q0w + 16 * qt + r, Sq - 1);
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds)
      qf[ds][qt] = *reinterpret_cast<const u32x4_t*>(qg + (int64_t)qrow * D + ds * 32 + g * 8);
  }

  float m_run[QT], l_run[QT];
  f32x4_t ot[DT][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) ot[dt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int kv_end = p.causal ? min(Skv, q0 + BQ) : Skv;
  const int nblk = (kv_end + KB - 1) / KB;

  auto compute = [&](int s, int blk) {
    const int kv0 = blk * KB;
    // a wave whose queries all precede the block sees only masked keys
    if (p.causal && kv0 > q0w + 16 * QT - 1) return;
    const lds_char_t* ks = stK(s);
    const lds_char_t* vs = stV(s);
    // ---- S^T = K^T Q^T; st[jt][qt][i] = score of key kv0 + 16 jt + 4 g + i
    f32x4_t st[4][QT];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) st[jt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds) {
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int d = ds * 32 + g * 8 + a4;                 // & 3 == a4
        const int ch = (2 * jt + (c4 >> 1)) ^ (2 * a4);
        const lds_char_t* q = ks + d * (KB * 2) + ch * 16 + (c4 & 1) * 8;
        const u32x2_t lo = lds_read_tr16(q);
        const u32x2_t hi = lds_read_tr16(q + 4 * (KB * 2));
        const u32x4_t kf = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) st[jt][qt] = mfma16(kf, qf[ds][qt], st[jt][qt]);
      }
    }
    // ---- masking (only blocks that reach past Skv or the diagonal)
    const bool edge = kv0 + KB > Skv || (p.causal && kv0 + KB - 1 > q0w);
    if (edge) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int qrow = q0w + 16 * qt + r;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kv0 + 16 * jt + 4 * g + i;
            if (key >= Skv || (p.causal && key > qrow)) st[jt][qt][i] = -INFINITY;
          }
      }
    }
    // ---- online softmax, log2 domain, lazy rescale
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[jt][qt][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mblk = mx * p.c2;
      if (__builtin_amdgcn_ballot_w64(mblk > m_run[qt] + 8.f) != 0) {
        const float m_new = fmaxf(m_run[qt], mblk);
        const float alpha = fast_exp2(m_run[qt] - m_new);   // 0 on the first visible block
        m_run[qt] = m_new;
        l_run[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) ot[dt][qt] *= alpha;
      }
      // rows that have seen no key keep m = -inf: exponentiate against 0
      const float mb = m_run[qt] == -INFINITY ? 0.f : m_run[qt];
      float ls = 0.f;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = fast_exp2(__builtin_fmaf(st[jt][qt][i], p.c2, -mb));
          st[jt][qt][i] = pv;
          ls += pv;
        }
      l_run[qt] += ls;
    }
    // ---- O^T += V^T P^T, 32 keys (tiles j0 = 2 pp, j1 = 2 pp + 1) per step
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      u32x4_t pf[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
        pf[qt] = u32x4_t{pack_bf16x2(st[2 * pp][qt][0], st[2 * pp][qt][1]),
                         pack_bf16x2(st[2 * pp][qt][2], st[2 * pp][qt][3]),
                         pack_bf16x2(st[2 * pp + 1][qt][0], st[2 * pp + 1][qt][1]),
                         pack_bf16x2(st[2 * pp + 1][qt][2], st[2 * pp + 1][qt][3])};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int ch = (2 * dt + (c4 >> 1)) ^ (2 * a4);
        const int k0r = 32 * pp + 4 * g + a4;               // & 3 == a4
        const lds_char_t* q = vs + k0r * VROW + ch * 16 + (c4 & 1) * 8;
        const u32x2_t lo = lds_read_tr16(q);                // keys 32pp + 4g + 0..3
        const u32x2_t hi = lds_read_tr16(q + 16 * VROW);    // keys 32pp + 16 + 4g + 0..3
        const u32x4_t vf = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) ot[dt][qt] = mfma16(vf, pf[qt], ot[dt][qt]);
      }
    }
  };

  // ---- pipeline: NS stages, waits placed by hand (see gemm.hip)
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nblk) issue(s, s);
  for (int it0 = 0; it0 < nblk; it0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int it = it0 + s;
      if (it < nblk) {
        const int younger = min(NS - 2, nblk - 1 - it);
        if (younger >= 2) LOOM_WAIT_VMCNT(2 * LPW);
        else if (younger == 1) LOOM_WAIT_VMCNT(LPW);
        else LOOM_WAIT_VMCNT(0);
        barrier_nofence();
        if (it + NS - 1 < nblk) issue((s + NS - 1) % NS, it + NS - 1);
        compute(s, it);
      }
    }
  }

  // ---- out = acc / l; ot[dt][qt][i] is d = 16 dt + 4 g + i of query q0w + 16 qt + r
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    __builtin_amdgcn_sched_barrier(0);
    float l = l_run[qt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.f / l;
    const int qrow = q0w + 16 * qt + r;
    if (qrow < Sq) {
      uint16_t* orow = p.out + ((int64_t)bh * Sq + qrow) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4_t o = ot[dt][qt];
        *reinterpret_cast<u32x2_t*>(orow + dt * 16 + 4 * g) =
            u32x2_t{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
      }
    }
  }
}

template <int D, int QT>
void launch_attn(const AttnParams& p, hipStream_t st) {
  hipLaunchKernelGGL((attention_kernel<D, QT>), dim3((unsigned)(p.BH * p.nqt)),
                     dim3(64 * kWaves), 0, st, p);
}

}  // namespace

extern "C" {

int loom_hip_attention(const void* k, const void* v, const void* q, void* out, int64_t BH,
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
  if (!(tile_m == 64 || tile_m == 128 || tile_m == 192 || tile_m == 256))
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "attention: tile_m %lld not built for gfx950 (64, 128, 192, 256)",
                     (long long)tile_m);
  if (!(D == 64 || D == 128))
    return loom_fail(err, errlen, LOOM_EUNSUP, "attention: head_dim %lld not built (64, 128)",
                     (long long)D);
  if (Skv % 8 != 0)
    return loom_fail(err, errlen, LOOM_EUNSUP, "attention: Skv must be a multiple of 8");
  if (!aligned16(k) || !aligned16(v) || !aligned16(q) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return loom_fail(err, errlen, LOOM_EINVAL, "attention: tensors must be 16-byte aligned");
  if (Sq > (1 << 30) || Skv > (1 << 30) || BH * cdiv64(Sq, tile_m) > 0x7fffffff)
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
  p.c2 = scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
#ifdef LOOM_ATTN_LEGACY
  if (D == 128) {
    if (tile_m == 128) launch_attn<128, 2>(p, st); else launch_attn<128, 1>(p, st);
  } else {
    if (tile_m == 128) launch_attn<64, 2>(p, st); else launch_attn<64, 1>(p, st);
  }
#else
  {
    const dim3 grid((unsigned)(p.BH * p.nqt)), block(256);
    switch ((D == 128 ? 10 : 0) + (int)(tile_m / 64)) {
      case 11: hipLaunchKernelGGL((attention_dma_kernel<128, 1>), grid, block, 0, st, p); break;
      case 12: hipLaunchKernelGGL((attention_dma_kernel<128, 2>), grid, block, 0, st, p); break;
      case 13: hipLaunchKernelGGL((attention_dma_kernel<128, 3>), grid, block, 0, st, p); break;
      case 14: hipLaunchKernelGGL((attention_dma_kernel<128, 4>), grid, block, 0, st, p); break;
      case 1: hipLaunchKernelGGL((attention_dma_kernel<64, 1>), grid, block, 0, st, p); break;
      case 2: hipLaunchKernelGGL((attention_dma_kernel<64, 2>), grid, block, 0, st, p); break;
      case 3: hipLaunchKernelGGL((attention_dma_kernel<64, 3>), grid, block, 0, st, p); break;
      default: hipLaunchKernelGGL((attention_dma_kernel<64, 4>), grid, block, 0, st, p); break;
    }
  }
#endif
  return loom_check_launch(err, errlen, "attention");
}

}  // extern "C"
