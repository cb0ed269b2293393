// decode.hip -- @flash_decode: multi-query split-KV decode on gfx950.
//
// Reference: examples/mqa_decode/IR/00_from_helion_frontend.mlir:6-202.
//   k [B, D, S] (keys transposed), v [B, S, D], q [B, H, D], out [B, H, D];
//   the H query heads of a batch share its single KV head.
//   Split s covers keys [s*tile_s, (s+1)*tile_s) with an online softmax
//   (:30-122), then lse_s = log(l) + m (:123-132) and o_s = acc / l
//   (:133-138) are gathered at index s (:139-146); split 0 combines
//   (:147-199): M = max_s lse_s, w_s = exp(lse_s - M) / sum exp(. - M),
//   out = sum_s w_s o_s.
//
// gfx950 mapping.  Decode is bound by streaming K and V from HBM; the 32
// heads sharing the KV head give 32 FLOP per KV byte, which at 8 TB/s is
// more arithmetic than the fp32 VALU peak, so S^T = K^T . Q^T and
// O^T += V^T . P^T run on MFMA and the kernel stays bound by the stream.
// One workgroup (4 waves) per (batch, split, group of 32 query heads):
//   - decode_dma_kernel (S a multiple of 8, or any S above D 128 or 32
//     heads with K staged through registers; 4 waves for up to 32 heads, 8
//     for 64): K and V stream through a ring of LDS-DMA stages (four, two at
//     D 256) and reach the MFMAs by transposed LDS reads (described at the
//     kernel);
//   - decode_split_kernel (other S, up to 32 heads and D 128): raw buffer loads straight into
//     registers, MFMA operands built by register transposes (v_perm_b32),
//     keys permuted inside a block and the permutation undone only where
//     results are addressed (softmax and P.V do not depend on key order).
// Softmax runs in the log2 domain in fp32.  The waves' partial states merge
// through LDS into (lse_s, o_s), exactly the reference's gathered tensors;
// decode_combine_kernel performs the split-0 combine.
// Any head dim that is a multiple of 8 up to 128 runs on the kernels built
// for 64 or 128, and up to 256 on the LDS-DMA kernel built for 256: K rows
// and q elements past it are zeros (copied from zeros, or read past the
// buffer range), so the scores are exact, and V columns past it only reach O
// columns that are never stored.
#include "common.h"

#include <cmath>
#include <mutex>

namespace {

constexpr int kWaves = 4;
constexpr int kBlockKeys = 64;    // keys per wave block: 16 lanes x 4 keys

struct DecodeParams {
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* q;
  float* lse;  // [ns, B, H]
  float* o;    // [ns, B, H, D]
  uint16_t* out;
  int B, H, S, tile_s, ns;
  int D;       // head dim: a multiple of 8, at most the kernel's D
  float c2;    // scale * log2(e)
};

// Split-0 combine of the reference (:147-199): M = max_s lse_s,
// w_s = exp(lse_s - M) / sum_s exp(lse_s - M), out = sum_s w_s o_s (ascending
// s).  One thread per two consecutive d of one (b, head): every split's lse
// and o loads are independent and issued together (in chunks of CH splits:
// 8 when there are at most 8, else 16), so the combine costs about one
// memory round trip.
template <bool F16, int CH>
__global__ void __launch_bounds__(256) decode_combine_kernel(DecodeParams p) {
  const int D = p.D;
  const int TPR = D / 2;       // threads per (b, head) row
  const int64_t BH = (int64_t)p.B * p.H;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t bh = t / TPR;
  if (bh >= BH) return;
  const int d = (int)(t % TPR) * 2;
  const int ns = p.ns;
  // every load of a chunk of CH splits is issued before any is used; across
  // chunks the running max moves and the sums rescale (one chunk at BASELINE
  // shapes, so one memory round trip)
  float M = -INFINITY, den = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c0 = 0; c0 < ns; c0 += CH) {
    float l[CH];
    f32x2_t o[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int64_t s = min(c0 + u, ns - 1);   // clamped: weight 0 past the end
      l[u] = p.lse[s * BH + bh];
      o[u] = *reinterpret_cast<const f32x2_t*>(p.o + (s * BH + bh) * D + d);
    }
    float mc = M;
#pragma unroll
    for (int u = 0; u < CH; ++u) mc = fmaxf(mc, l[u]);
    const float r = expf(M - mc);   // 0 on the first chunk (M = -inf)
    den *= r;
    a0 *= r;
    a1 *= r;
    M = mc;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const float w = c0 + u < ns ? expf(l[u] - M) : 0.f;
      den += w;
      a0 += w * o[u][0];
      a1 += w * o[u][1];
    }
  }
  const float inv = 1.f / den;
  *reinterpret_cast<uint32_t*>(p.out + bh * D + d) = pack2<F16>(a0 * inv, a1 * inv);
}

// ---------------------------------------------------------------------------
// Split kernel, LDS-DMA form (the production path: S a multiple of 8).  One
// workgroup of four waves per (batch, split, group of up to 32 query heads).
// K and V of the split stream through LDS in 64-key stages copied by LDS DMA
// (global_load_lds_dwordx4), three stages deep up to D 128 (two 64 KB stages
// at D 256): 64 KB per workgroup in flight with no registers held by loads
// (a fourth stage, 96 KB in flight, streamed 2-3% slower at every shape
// measured; two stages, 32 KB, slower at the large ones).  Ks is [d][key]
// and Vs [key][d], as the tensors lay them
// out; the MFMA operands that need k-contiguous data come from
// ds_read_b64_tr_b16:
//   S^T[key, h]  = K^T . Q^T : row operand K^T from Ks (lane r: key, eight
//                              consecutive d), column operand Q^T (16 heads);
//   O^T[d, h]   += V^T . P^T : row operand V^T from Vs (lane r: d, keys
//                              4 g + 0..3 and 16 + 4 g + 0..3 of a 32-key half),
//                              the keys P^T holds in lane group g.
// Wave w takes the 32-key half kh = w & 1 of every stage for the heads of
// tile ht = w >> 1 (16 heads; 8 W head slots in all -- 32 with four waves,
// 64 with eight, which serve more heads per pass over K and V -- slots past
// H are zero queries and never stored), with an online softmax of its own in the log2
// domain whose base only moves when a score rises 8 above it (P <= 2^8; the
// row sum is an MFMA of the same bf16 P against ones, so numerator and
// denominator see identical weights).  At the end the two halves of each
// head tile merge through the (then idle) stage LDS into (lse_s, o_s).
// Blocks start at the split's first key rounded down to a multiple of 8;
// keys outside [s0, s1) are masked to -inf, reads past S are clamped.
// ---------------------------------------------------------------------------
// 16-byte chunk swizzles of the Ks and Vs rows, as in attention.hip: the
// banks repeat every 256 bytes, and each 32-lane pass of a transposed read
// must touch distinct ones.  Ks (128-byte rows): rows d, d^2, d^8, d^10 share
// a window position.  Vs: D 128 (256-byte rows) all eight rows of a pass, D 64
// rows r, r^2, r^4, r^6.
LOOM_DEV int dk_swz(int d) { return (2 * (d & 3)) ^ (2 * ((d >> 3) & 1)); }
template <int D>
LOOM_DEV int dv_swz(int k) { return D >= 128 ? 2 * (k & 7) : 2 * ((k >> 1) & 3); }

// KREG (S not a multiple of 8): K rows [d][0..S) do not start on 16-byte
// boundaries, so K cannot be copied by 16-byte LDS DMA.  Each lane then
// loads its 16-byte pieces of a K block into registers (row_piece8), issued
// before the block NS-1 stages ahead of the one being computed and written to
// the DMA's LDS positions after that computation; V keeps its DMA.
// NSX: stages when nonzero (2: a grid above one workgroup per CU then fits
// two per CU), else three up to D 128 and two (64 KB each) at D 256
template <int D, bool F16, bool KREG, int W, int NSX = 0>
__global__ void __launch_bounds__(64 * W) decode_dma_kernel(DecodeParams p) {
  constexpr int KB = 64;                       // keys per stage
  constexpr int NS = NSX ? NSX : (D > 128 ? 2 : 3);
  constexpr int HS = 8 * W;                    // head slots (16 per pair of waves)
  constexpr int K_BYTES = D * KB * 2, V_BYTES = KB * D * 2;
  constexpr int K_INSTR = K_BYTES / 1024 / W, V_INSTR = V_BYTES / 1024 / W;
  constexpr int LPW = K_INSTR + V_INSTR;       // DMA instructions per wave per stage
  constexpr int VROW = D * 2, V_ROWS_PER_I = 1024 / VROW;
  constexpr int DSTEPS = D / 32, DT = D / 16;
  static_assert(LPW * (NS - 2) <= 63, "vmcnt range");
  constexpr int STAGE = K_BYTES + V_BYTES;
  constexpr int ROW = D + 4;                   // merge row: D o values, m, l (16-byte rows)
  constexpr int MERGE = W * 16 * ROW * 4;      // per wave: 16 heads
  constexpr int Q_BYTES = HS * D * 2;          // the head slots of q
  // the merge reuses the stage ring and, past it, the q slots (read into
  // registers at the first block)
  static_assert(MERGE <= NS * STAGE + Q_BYTES, "merge area fits the LDS");
  constexpr int Q_INSTR = Q_BYTES / 1024 / W;
  __shared__ __attribute__((aligned(1024))) char smem[NS * STAGE + Q_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int a4 = r >> 2, c4 = r & 3;           // transposed-read lane roles
  const int kh = wave & 1, ht = wave >> 1;

  const int split = blockIdx.x, b = blockIdx.y;
  const int H = p.H, S = p.S;
  // head group blockIdx.z: query heads h0 .. h0 + Hl - 1 (HS head slots)
  const int h0 = (int)blockIdx.z * HS, Hl = min(HS, H - h0);
  const int s0 = split * p.tile_s;
  const int s1 = min(S, s0 + p.tile_s);
  const int kbeg = s0 & ~7;                    // 16-byte aligned first key
  const int nblk = (s1 - kbeg + KB - 1) / KB;
  const int Dr = p.D;
  const uint16_t* __restrict__ kg = p.k + (int64_t)b * Dr * S;
  const uint16_t* __restrict__ vg = p.v + (int64_t)b * S * Dr;

  auto stK = [&](int s) { return (lds_char_t*)(smem + s * STAGE); };
  auto stV = [&](int s) { return (lds_char_t*)(smem + s * STAGE + K_BYTES); };
  // ---- DMA of block `blk` into stage s (reads past S clamped; masked
  // later; Ks rows d >= Dr, eight to a copy, come from zeros; Vs chunks past
  // Dr repeat the row's last chunk)
  auto issue = [&](int s, int blk) {
    const int kv0 = kbeg + blk * KB;
    const uint32_t lk = lds_addr(stK(s)), lv = lds_addr(stV(s));
    if constexpr (!KREG) {
#pragma unroll
      for (int i = 0; i < K_INSTR; ++i) {
        const int j = wave * K_INSTR + i;
        const int d = j * 8 + lane / 8;                 // Ks row
        const int c = (lane % 8) ^ dk_swz(d);
        const int key = min(kv0 + c * 8, S - 8);
        if (j * 8 < Dr)                                 // wave-uniform
          dma_load16(kg + (int64_t)d * S + key, lk + j * 1024);
        else
          dma_load16(loom_zero_kb + lane * 4, lk + j * 1024);
      }
    }
#pragma unroll
    for (int i = 0; i < V_INSTR; ++i) {
      const int j = wave * V_INSTR + i;
      const int kr = j * V_ROWS_PER_I + lane / (D / 8); // Vs row (key)
      const int c = min((lane % (D / 8)) ^ dv_swz<D>(kr), Dr / 8 - 1);
      const int key = min(kv0 + kr, S - 1);
      dma_load16(vg + (int64_t)key * Dr + c * 8, lv + j * 1024);
    }
  };
  // ---- KREG: this lane's K pieces of block `blk` (the DMA's positions: row
  // d, 8 keys from kv0 + 8 c) into registers, then into stage s.  Pieces
  // past S read as zeros (their keys are masked); k needs 2-byte alignment.
  const rsrc_t krs = make_rsrc(kg, KREG ? (uint32_t)(Dr * S * 2) : 0u);
  u32x4_t kr[KREG ? K_INSTR : 1];
  auto kload = [&](int blk) {
    const int kv0 = kbeg + blk * KB;
#pragma unroll
    for (int i = 0; i < K_INSTR; ++i) {
      const int j = wave * K_INSTR + i;
      const int d = j * 8 + lane / 8;
      const int c = (lane % 8) ^ dk_swz(d);
      kr[i] = j * 8 < Dr ? row_piece8(krs, S, d, kv0 + c * 8)   // padding rows: zeros
                         : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto kstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < K_INSTR; ++i)
      *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(
          stK(s) + (wave * K_INSTR + i) * 1024 + lane * 16) = kr[i];
  };

  // q[b] (the group's head slots, rows past its heads clamped to its last
  // head and zeroed on read, as are the elements past Dr)
  // arrives by LDS DMA ahead of the first stages: a plain load would make the
  // compiler wait for every copy in flight before its first use
  lds_char_t* sq = (lds_char_t*)(smem + NS * STAGE);
#pragma unroll
  for (int i = 0; i < Q_INSTR; ++i) {
    const int j = wave * Q_INSTR + i;
    const int e = j * 512 + lane * 8;                     // element of the [HS][D] slots
    const int hq = h0 + min(e / D, Hl - 1);
    dma_load16(p.q + ((int64_t)b * H + hq) * Dr + min(e % D, Dr - 8), lds_addr(sq) + j * 1024);
  }
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nblk) {
      if constexpr (KREG) {
        kload(s);
        kstore(s);
      }
      issue(s, s);
    }

  // Q^T operand of this wave's head tile, q[b][16 ht + r][32 ds + 8 g ..],
  // read from LDS once the first stage has landed
  const int h = 16 * ht + r;
  u32x4_t qf[DSTEPS];

  const float c2 = p.c2;
  float m_run = 0.f;                           // base (log2 domain) of head h
  f32x4_t ot[DT], lacc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) ot[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u32x4_t ones = u32x4_t{kOnePair<F16>, kOnePair<F16>, kOnePair<F16>, kOnePair<F16>};
  bool first = true;

  auto compute = [&](int s, int blk) {
    const int kv0 = kbeg + blk * KB + 32 * kh;   // this wave's 32 keys
    const lds_char_t* ks = stK(s);
    const lds_char_t* vs = stV(s);
    // ---- raw scores S^T = K^T Q^T; st[j][i] is key kv0 + 16 j + 4 g + i of head h
    f32x4_t st[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) st[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int jt = 2 * kh + j;
        const int d = ds * 32 + g * 8 + a4;
        const int ch = (2 * jt + (c4 >> 1)) ^ dk_swz(d);
        const lds_char_t* q = ks + d * (KB * 2) + ch * 16 + (c4 & 1) * 8;
        const u32x2_t lo = lds_read_tr16(q);
        const u32x2_t hi = lds_read_tr16(q + 4 * (KB * 2));
        st[j] = mfma16t<F16>(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, qf[ds], st[j]);
      }
    }
    // ---- log2-domain scores relative to the base; keys outside the split
    // (or past S) are -inf
    const bool edge = kv0 < s0 || kv0 + 32 > s1;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = __builtin_fmaf(st[j][i], c2, -m_run);
        if (edge) {
          const int key = kv0 + 16 * j + 4 * g + i;
          if (key < s0 || key >= s1) v = -INFINITY;
        }
        st[j][i] = v;
      }
    // ---- lazy online softmax: the base moves (and O, l rescale) only on
    // this wave's first block or when a score rises more than 8 above it
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[j][i]);
    if (first || __builtin_amdgcn_ballot_w64(mx > 8.f) != 0) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // masking is per key, so a block is masked for every head or for none:
      // a wholly masked first block adds nothing and leaves the base unset
      if (first && __builtin_amdgcn_ballot_w64(mx != -INFINITY) == 0) return;
      const float shift = first ? mx : fmaxf(mx, 0.f);
      if (!first) {
        const float alpha = fast_exp2(-shift);
        lacc *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) ot[dt] *= alpha;
      }
      m_run += shift;
#pragma unroll
      for (int j = 0; j < 2; ++j) st[j] -= shift;
      first = false;
    }
    f32x4_t e0, e1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e0[i] = fast_exp2(st[0][i]);
      e1[i] = fast_exp2(st[1][i]);
    }
    const u32x4_t pf = u32x4_t{pack2<F16>(e0[0], e0[1]), pack2<F16>(e0[2], e0[3]),
                               pack2<F16>(e1[0], e1[1]), pack2<F16>(e1[2], e1[3])};
    lacc = mfma16t<F16>(ones, pf, lacc);
    // ---- O^T += V^T P^T over the 32 keys
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int k0r = 32 * kh + 4 * g + a4;
      const int ch = (2 * dt + (c4 >> 1)) ^ dv_swz<D>(k0r);
      const lds_char_t* q = vs + k0r * VROW + ch * 16 + (c4 & 1) * 8;
      const u32x2_t lo = lds_read_tr16(q);                // keys 4 g + 0..3
      const u32x2_t hi = lds_read_tr16(q + 16 * VROW);    // keys 16 + 4 g + 0..3
      ot[dt] = mfma16t<F16>(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pf, ot[dt]);
    }
  };

  // ---- pipeline: NS stages, the first NS-1 issued above; each wave waits
  // for its own copies of the stage (copies complete in issue order, q's
  // first), the barrier for everyone's (the waits are placed by hand, as in
  // gemm.hip and attention.hip)
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
        if (it == 0) {
          // q's copies were issued before stage 0's, so they have landed too
#pragma unroll
          for (int ds = 0; ds < DSTEPS; ++ds) {
            const u32x4_t raw = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                sq + (h * D + ds * 32 + g * 8) * 2);
            qf[ds] = h < Hl && ds * 32 + g * 8 < Dr ? raw : u32x4_t{0u, 0u, 0u, 0u};
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

  // ---- merge the two key halves of each head tile through LDS: per wave
  // [16 heads][ROW] (fp32)
  LOOM_WAIT_VMCNT(0);
  barrier_nofence();
  float* mg = reinterpret_cast<float*>(smem);
  float* my = mg + wave * 16 * ROW + r * ROW;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) my[dt * 16 + 4 * g + i] = ot[dt][i];
  if (g == 0) {
    my[D] = m_run;
    my[D + 1] = lacc[0];
  }
  __syncthreads();
  // one head and D/8 consecutive d per thread: the weights once, then
  // 16-byte LDS reads and stores
  constexpr int DPT = D / 8;                   // d values per thread
  const int hh = tid >> 3, d0 = (tid & 7) * DPT;
  if (hh < Hl) {
    const float* w0 = mg + (2 * (hh >> 4)) * 16 * ROW + (hh & 15) * ROW;
    const float* w1 = w0 + 16 * ROW;
    // a half that saw no key of the split (l = 0) takes no part
    const float l0 = w0[D + 1], l1 = w1[D + 1];
    const float M = l0 > 0.f ? (l1 > 0.f ? fmaxf(w0[D], w1[D]) : w0[D]) : w1[D];
    const float f0 = l0 > 0.f ? fast_exp2(w0[D] - M) : 0.f;
    const float f1 = l1 > 0.f ? fast_exp2(w1[D] - M) : 0.f;
    const float L = l0 * f0 + l1 * f1;
    const float g0 = f0 / L, g1 = f1 / L;
    const int64_t row = ((int64_t)split * p.B + b) * H + h0 + hh;
    f32x4_t* dst = reinterpret_cast<f32x4_t*>(p.o + row * Dr + d0);
#pragma unroll
    for (int u = 0; u < DPT / 4; ++u) {
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(w0 + d0 + 4 * u);
      const f32x4_t c = *reinterpret_cast<const f32x4_t*>(w1 + d0 + 4 * u);
      if (d0 + 4 * u < Dr) dst[u] = a * g0 + c * g1;
    }
    if (d0 == 0) p.lse[row] = (logf(L) + M * 0.69314718055994530942f);
  }
}

// K rows start at 2-byte granularity here (S not a multiple of 8), and each
// lane's four keys of a row are one 8-byte buffer load at a 2-, 4- or 8-byte
// aligned offset.  That relies on the unaligned access mode ROCm's driver
// sets for every GPU process (SH_MEM_CONFIG.alignment_mode UNALIGNED: dword
// and wider loads take any byte address); the parity tests at odd S and odd
// tile_s pin it.  A load reaching past the buffer's range returns zeros
// whole, valid bytes included, so rows that can hold K's last keys keep one
// 2-byte load per key (tests/test_gpu_head_dims.py puts the deciding keys
// there).
template <int D, int HT, bool F16>
__global__ void __launch_bounds__(64 * kWaves) decode_split_kernel(DecodeParams p) {
  constexpr int VEC = D / 16;     // d values per lane per V row, also # of d tiles
  constexpr int DSTEPS = D / 32;  // 32-deep MFMA steps over d
  constexpr int NSTEPS = DSTEPS + 2;
  // ring slots: three (loads two steps ahead) where they divide the step
  // count, else two
  constexpr int R = NSTEPS % 3 == 0 ? 3 : 2;
  static_assert(NSTEPS % R == 0, "ring must divide the step count");
  constexpr int HP = HT * 16;     // padded head count
  constexpr int ACC_STRIDE = D + 1;
  __shared__ float sm_m[kWaves][HP];
  __shared__ float sm_l[kWaves][HP];
  __shared__ float sm_acc[kWaves][HP * ACC_STRIDE];

  const int split = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int H = p.H, S = p.S;
  // head group blockIdx.z: query heads h0 .. h0 + Hl - 1
  const int h0 = (int)blockIdx.z * 32, Hl = min(32, H - h0);
  const int s0 = split * p.tile_s;
  const int s1 = min(S, s0 + p.tile_s);
  const int nblk = (s1 - s0 + kBlockKeys - 1) / kBlockKeys;

  // K rows past Dr lie past the descriptor's range: they read as zeros
  const int Dr = p.D;
  const rsrc_t krs = make_rsrc(p.k + (int64_t)b * Dr * S, (uint32_t)(Dr * S * 2));
  const rsrc_t vrs = make_rsrc(p.v + (int64_t)b * S * Dr, (uint32_t)(S * Dr * 2));
  const uint16_t* __restrict__ qb = p.q + ((int64_t)b * H + h0) * Dr;

  // Q^T operands, shared by the waves through LDS: slot [ds][ht][lane]
  // holds q[h = r + 16 ht][32 ds + 8 g .. +7]
  __shared__ u32x4_t sm_q[DSTEPS][HT][64];
  for (int e = threadIdx.x; e < DSTEPS * HT * 64; e += 64 * kWaves) {
    const int ln = e & 63, ht = (e >> 6) % HT, ds = (e >> 6) / HT;
    const int h = (ln & 15) + 16 * ht, d0 = ds * 32 + (ln >> 4) * 8;
    sm_q[ds][ht][ln] = h < Hl && d0 < Dr
                           ? *reinterpret_cast<const u32x4_t*>(qb + (int64_t)h * Dr + d0)
                           : u32x4_t{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // ---- loads of step `st` of the block starting at key `base`.  A block
  // this wave does not have (valid false) is still issued, at an offset
  // past the descriptor's range (zeros, no memory access): with every load
  // unconditional the compiler waits only for the loads it needs, not for
  // the ones in flight ahead of them.
  constexpr uint32_t kNone = 0x7ffffff0u;
  auto issue = [&](int base, int st, u32x4_t (&buf)[8], bool valid) {
    if (st < DSTEPS) {
      // K rows d = 32 st + 8 g + e, keys base + 4 r .. +3
      const uint32_t off = ((uint32_t)(st * 32 + g * 8) * S + base + r * 4) * 2;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t o = valid ? off + (uint32_t)(e * S) * 2 : kNone;
        if (e < 7) {
          const u32x2_t w = buf_load8(krs, o);
          buf[e] = u32x4_t{w[0], w[1], 0u, 0u};
        } else {
          // rows 8 m + 7 hold the last row of K (D is a multiple of 8),
          // whose pieces can reach past the tensor's end: a load that does
          // returns zeros whole, so these take one 2-byte load per key
          uint32_t h[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) h[x] = buf_load2(krs, o + 2 * x);
          buf[e] = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), 0u, 0u};
        }
      }
    } else {
      // V rows for 32-key step c: slot t holds key base + 16 g + 4 (t%4) + 2c + t/4
      const int c = st - DSTEPS;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int key = base + 16 * g + 4 * (t & 3) + 2 * c + (t >> 2);
        const uint32_t o = valid ? ((uint32_t)key * Dr + r * VEC) * 2 : kNone;
        if constexpr (VEC == 8) {
          buf[t] = buf_load16(vrs, o);
        } else {
          const u32x2_t w = buf_load8(vrs, o);
          buf[t] = u32x4_t{w[0], w[1], 0u, 0u};
        }
      }
    }
  };

  float m_run[HT], l_run[HT];
  f32x4_t ot[VEC][HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    m_run[ht] = -INFINITY;
    l_run[ht] = 0.f;
#pragma unroll
    for (int u = 0; u < VEC; ++u) ot[u][ht] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // loads run R-1 steps ahead of the math (into the wave's next block at the
  // end of one)
  u32x4_t ring[R][8];
#pragma unroll
  for (int a = 0; a < R - 1; ++a) issue(s0 + wave * kBlockKeys, a, ring[a], wave < nblk);

  for (int bi = wave; bi < nblk; bi += kWaves) {
    const int base = s0 + bi * kBlockKeys;
    const bool has_next = bi + kWaves < nblk;
    const int next_base = base + kWaves * kBlockKeys;
    f32x4_t st_acc[4][HT];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) st_acc[j][ht] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int st = 0; st < NSTEPS; ++st) {
      // prefetch R-1 steps ahead (into the next block near the end)
      if (st + R - 1 < NSTEPS)
        issue(base, st + R - 1, ring[(st + R - 1) % R], true);
      else
        issue(next_base, st + R - 1 - NSTEPS, ring[(st + R - 1) % R], has_next);

      u32x4_t (&cur)[8] = ring[st % R];
      if (st < DSTEPS) {
        // ---- S^T += K^T Q^T for d rows 32 st .. +31; kt[j] = d values
        // 32st+8g..+7 of key base + 4r + j (8x4 transpose of 16-bit values)
        u32x4_t kt[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t x = cur[2 * i][j / 2], y = cur[2 * i + 1][j / 2];
            kt[j][i] = (j & 1) ? pack_hi(x, y) : pack_lo(x, y);
          }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ht = 0; ht < HT; ++ht)
            st_acc[j][ht] = mfma16t<F16>(kt[j], sm_q[st][ht][lane], st_acc[j][ht]);
      }
      if (st == DSTEPS - 1) {
        // ---- online softmax (log2 domain); st_acc[j][ht][i] is the score of
        // key base + 16 g + 4 i + j for head r + 16 ht
        if (base + kBlockKeys > s1) {  // keys past the split end: -inf
#pragma unroll
          for (int ht = 0; ht < HT; ++ht)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (base + 16 * g + 4 * i + j >= s1) st_acc[j][ht][i] = -INFINITY;
        }
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          // max of the raw scores; scale > 0 commutes with max
          float mx = -INFINITY;
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st_acc[j][ht][i]);
          mx = fmaxf(mx, __shfl_xor(mx, 16));
          mx = fmaxf(mx, __shfl_xor(mx, 32));
          const float m_new = fmaxf(m_run[ht], mx * p.c2);
          const float alpha = fast_exp2(m_run[ht] - m_new);
          m_run[ht] = m_new;
          float ls = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float pv = fast_exp2(__builtin_fmaf(st_acc[j][ht][i], p.c2, -m_new));
              st_acc[j][ht][i] = pv;
              ls += pv;
            }
          l_run[ht] = l_run[ht] * alpha + ls;
#pragma unroll
          for (int u = 0; u < VEC; ++u) ot[u][ht] *= alpha;
        }
      }
      if (st >= DSTEPS) {
        // ---- O^T += V^T P^T over keys of tiles j0 = 2c, j1 = 2c + 1
        const int c = st - DSTEPS, j0 = 2 * c, j1 = 2 * c + 1;
        u32x4_t pf[HT];
#pragma unroll
        for (int ht = 0; ht < HT; ++ht)
          pf[ht] = u32x4_t{pack2<F16>(st_acc[j0][ht][0], st_acc[j0][ht][1]),
                           pack2<F16>(st_acc[j0][ht][2], st_acc[j0][ht][3]),
                           pack2<F16>(st_acc[j1][ht][0], st_acc[j1][ht][1]),
                           pack2<F16>(st_acc[j1][ht][2], st_acc[j1][ht][3])};
        // transpose: va[u] = V[key_t][VEC r + u] for slots t = 0..7
        u32x4_t va[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t x = cur[2 * i][u / 2], y = cur[2 * i + 1][u / 2];
            va[u][i] = (u & 1) ? pack_hi(x, y) : pack_lo(x, y);
          }
#pragma unroll
        for (int u = 0; u < VEC; ++u)
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) ot[u][ht] = mfma16t<F16>(va[u], pf[ht], ot[u][ht]);
      }
    }
  }

  // ---- per-wave state to LDS: row sums reduced over the 4 lane groups
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    float l = l_run[ht];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int h = r + 16 * ht;
    if (g == 0) {
      sm_m[wave][h] = m_run[ht];
      sm_l[wave][h] = l;
    }
    // ot[u][ht][i]: d = VEC*(4g + i) + u, head h
#pragma unroll
    for (int u = 0; u < VEC; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm_acc[wave][h * ACC_STRIDE + VEC * (4 * g + i) + u] = ot[u][ht][i];
  }
  __syncthreads();

  // ---- merge the waves: (lse_s, o_s) for every (head, d) of this split
  const int64_t row0 = ((int64_t)split * p.B + b) * H + h0;
  for (int e = threadIdx.x; e < Hl * Dr; e += 64 * kWaves) {
    const int h = e / Dr, d = e % Dr;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w][h] - M);  // 0 for a wave that saw no key
      L += sm_l[w][h] * f;
      o += sm_acc[w][h * ACC_STRIDE + d] * f;
    }
    p.o[(row0 + h) * Dr + d] = o / L;
    if (d == 0) p.lse[row0 + h] = logf(L) + M * 0.69314718055994530942f;
  }

}

template <int D, int HT, bool F16>
void launch_split(const DecodeParams& p, hipStream_t st) {
  const dim3 grid(p.ns, p.B, (p.H + 31) / 32), block(64 * kWaves);
  hipLaunchKernelGGL((decode_split_kernel<D, HT, F16>), grid, block, 0, st, p);
}

template <int D, bool F16, int NSX>
void launch_dma_ns(const DecodeParams& p, bool kreg, bool wide, const dim3& grid, hipStream_t st) {
  if (wide) {   // three stages only (NSX 0)
    if (kreg) hipLaunchKernelGGL((decode_dma_kernel<D, F16, true, 8>), grid, dim3(512), 0, st, p);
    else hipLaunchKernelGGL((decode_dma_kernel<D, F16, false, 8>), grid, dim3(512), 0, st, p);
  } else {
    if (kreg) hipLaunchKernelGGL((decode_dma_kernel<D, F16, true, 4, NSX>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((decode_dma_kernel<D, F16, false, 4, NSX>), grid, dim3(256), 0, st, p);
  }
}

// Up to D 128 the 4-wave kernel's ring has three stages (64 KB in flight,
// one workgroup per CU by LDS) while the grid fits the CUs, and two when it
// has more workgroups than CUs, so that two fit per CU (72 KB of LDS and
// about 160 VGPRs each) and the grid runs in one round.  Graph of 20 calls,
// same run: B32 H32 D128 S8192 tile_s 1024 (256 workgroups) 30.0 us with
// three stages against 31.7 with two; tile_s 512 35.3 against 31.8;
// tile_s 256 44.1 against 38.5; B16 tile_s 256 23.4 against 20.8.  The
// 8-wave kernel's registers allow one workgroup per CU either way, so it
// keeps three stages.
template <int D, bool F16>
void launch_dma(const DecodeParams& p, bool kreg, bool wide, hipStream_t st) {
  const int hs = wide ? 64 : 32;
  const dim3 grid((unsigned)p.ns, (unsigned)p.B, (unsigned)((p.H + hs - 1) / hs));
  const int cus = stream_cus(st);
  const bool two = D <= 128 && !wide && cus > 0 && (int64_t)grid.x * grid.y * grid.z > cus;
  if (two) launch_dma_ns<D, F16, 2>(p, kreg, wide, grid, st);
  else launch_dma_ns<D, F16, 0>(p, kreg, wide, grid, st);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }




template <bool F16>
int flash_decode_impl(const void* k, const void* v, const void* q, void* out,
                          void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                          int64_t D, int64_t S, float scale, int64_t tile_b, int64_t tile_s,
                          int64_t tile_n, void* stream, char* err, size_t errlen) {
  if (!k || !v || !q || !out)
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: null tensor pointer");
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0)
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: extents must be positive");
  if (tile_b <= 0 || tile_s <= 0 || tile_n <= 0 || tile_b > B || tile_s > S || tile_n > S)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "flash_decode: tiles must satisfy 1 <= tile_b <= B, 1 <= tile_s, tile_n <= S "
                     "(tile_b=%lld tile_s=%lld tile_n=%lld)",
                     (long long)tile_b, (long long)tile_s, (long long)tile_n);
  // the running max is taken over raw scores and scaled afterwards, which
  // equals the max of the scaled scores only for a positive scale
  if (!(scale > 0.f) || !std::isfinite(scale))
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "flash_decode: scale must be finite and positive (got %g)", (double)scale);
  if (D % 8 != 0 || D > 256)
    return loom_fail(err, errlen, LOOM_EUNSUP,
                     "flash_decode: head_dim %lld not built (a multiple of 8 up to 256)",
                     (long long)D);
  if (H > 32 * 65535)
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: too many query heads (got %lld)",
                     (long long)H);
  if (!loom_prod_le({S, D, 2}, 0x7fffffffll) || B > 65535)
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: S*D or B too large");
  if (!aligned16(k) || !aligned16(v) || !aligned16(q) || !aligned16(out))
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: tensors must be 16-byte aligned");
  const int64_t ns = cdiv64(S, tile_s);
  const size_t need = loom_hip_flash_decode_workspace_bytes(B, H, D, S, tile_s);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "flash_decode: workspace needs %zu bytes (16-byte aligned), got %zu", need,
                     workspace_bytes);
  DecodeParams p{};
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q = static_cast<const uint16_t*>(q);
  p.lse = static_cast<float*>(workspace);
  const size_t lse_bytes = align256((size_t)ns * B * H * sizeof(float));
  p.o = reinterpret_cast<float*>(static_cast<char*>(workspace) + lse_bytes);
  p.out = static_cast<uint16_t*>(out);
  p.B = (int)B;
  p.H = (int)H;
  p.S = (int)S;
  p.tile_s = (int)tile_s;
  p.ns = (int)ns;
  p.D = (int)D;
  p.c2 = scale * 1.4426950408889634f;
  if (loom_validate_only()) return loom_ok(err, errlen);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the kernels built for 64, 128 or 256 (the next one up) run any narrower D
  const bool d128 = D > 64;
  // More than 32 query heads: 8-wave workgroups of 64 heads, so K and V are
  // streamed once per 64 heads, not per 32 (B32 H48 D128 S8192: 33.2 us
  // against 52.2).  S not a multiple of 8: the register kernel up to 32
  // heads and D 128 (B32 H32 D128 S8190: 35 us against 47 with K staged
  // through registers into the LDS-DMA kernel); that KREG form for more
  // heads (H48 S8191: 38.9 us against the register kernel's 60.1, which
  // takes 32 heads per pass) and above D 128, where the register kernel is
  // not built
  const bool kreg = S % 8 != 0;
  const bool wide = H > 32;
  if (!kreg || D > 128 || wide) {
    if (D > 128) launch_dma<256, F16>(p, kreg, wide, st);
    else if (d128) launch_dma<128, F16>(p, kreg, wide, st);
    else launch_dma<64, F16>(p, kreg, wide, st);
  } else {
    if (d128) {
      if (H > 16) launch_split<128, 2, F16>(p, st); else launch_split<128, 1, F16>(p, st);
    } else {
      if (H > 16) launch_split<64, 2, F16>(p, st); else launch_split<64, 1, F16>(p, st);
    }
  }
  int rc = loom_check_launch(err, errlen, "flash_decode (split)");
  if (rc) return rc;
  const dim3 cgrid((unsigned)cdiv64(B * H * D / 2, 256)), cblock(256);
  if (p.ns <= 8) hipLaunchKernelGGL((decode_combine_kernel<F16, 8>), cgrid, cblock, 0, st, p);
  else hipLaunchKernelGGL((decode_combine_kernel<F16, 16>), cgrid, cblock, 0, st, p);
  return loom_check_launch(err, errlen, "flash_decode (combine)");
}

// ---------------------------------------------------------------------------
// Allocation-free form (loom_hip_flash_decode_noalloc): the split partials go
// to `scratch`, a file-scope device array, instead of a caller workspace.
// Every device the library runs on holds its own copy until the process
// ends.  In host code `scratch` names a host-side stand-in, never device
// memory: its address on a device comes from hipGetSymbolAddress, taken once
// per device with that device current and kept in g_scratch.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)16 << 20;   // 16 MiB of split partials

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch[kMaxDevices];
hipError_t g_scratch_rc[kMaxDevices];
std::atomic<bool> g_scratch_ready[kMaxDevices];

// Device address of `scratch` on the device `stream` belongs to (the current
// device for the null stream).
int scratch_on(void* stream, void** ptr, char* err, size_t errlen) {
  int dev = 0;
  hipError_t e = hipSuccess;
  if (stream != nullptr) {
    hipDevice_t d = 0;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &d);
    dev = (int)d;
  } else {
    e = hipGetDevice(&dev);
  }
  if (e != hipSuccess)
    return loom_fail(err, errlen, LOOM_EHIP, "flash_decode_noalloc: no device for the stream: %s",
                     hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return loom_fail(err, errlen, LOOM_EUNSUP, "flash_decode_noalloc: device %d above %d", dev,
                     kMaxDevices - 1);
  // The address is looked up once per device, outside any graph capture: a
  // first call made while `stream` is being captured is refused (nothing is
  // recorded and nothing is cached, so a later call outside capture resolves
  // it and every call after that may be captured).
  if (!g_scratch_ready[dev].load(std::memory_order_acquire) && stream != nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) == hipSuccess &&
        cs != hipStreamCaptureStatusNone)
      return loom_fail(err, errlen, LOOM_EINVAL,
                       "flash_decode_noalloc: the first call on device %d must be made outside "
                       "graph capture (it looks up the scratch address)",
                       dev);
  }
  std::call_once(g_scratch_once[dev], [dev] {
    int cur = 0;
    hipError_t r = hipGetDevice(&cur);
    if (r == hipSuccess && cur != dev) r = hipSetDevice(dev);
    void* ptr = nullptr;
    if (r == hipSuccess) r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    g_scratch[dev] = ptr;
    g_scratch_rc[dev] = r;
    g_scratch_ready[dev].store(true, std::memory_order_release);
  });
  if (g_scratch_rc[dev] != hipSuccess || g_scratch[dev] == nullptr)
    return loom_fail(err, errlen, LOOM_EHIP,
                     "flash_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                     dev, hipGetErrorString(g_scratch_rc[dev]));
  *ptr = g_scratch[dev];
  return LOOM_OK;
}

}  // namespace

extern "C" {

int loom_hip_flash_decode_noalloc(const void* k, const void* v, const void* q, void* out,
                                  int64_t B, int64_t H, int64_t D, int64_t S, float scale,
                                  int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                  char* err, size_t errlen) {
  // every check of the workspace form first (validate-only, with a stand-in
  // workspace of the scratch's size), so a rejected call touches no device
  const size_t need = loom_hip_flash_decode_workspace_bytes(B, H, D, S, tile_s);
  if (need > kScratchBytes)
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "flash_decode_noalloc: the split partials need %zu bytes, the static scratch "
                     "holds %zu (fewer splits: a larger tile_s)",
                     need, kScratchBytes);
  bool& vo = loom_validate_only_flag();
  const bool outer = vo;
  vo = true;
  int rc = flash_decode_impl<false>(k, v, q, out, reinterpret_cast<void*>(uintptr_t(1) << 20),
                                    kScratchBytes, B, H, D, S, scale, tile_b, tile_s, tile_n,
                                    stream, err, errlen);
  vo = outer;
  if (rc || outer) return rc;
  void* ptr = nullptr;
  if ((rc = scratch_on(stream, &ptr, err, errlen))) return rc;
  return flash_decode_impl<false>(k, v, q, out, ptr, kScratchBytes, B, H, D, S, scale, tile_b,
                                  tile_s, tile_n, stream, err, errlen);
}

size_t loom_hip_flash_decode_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t S,
                                             int64_t tile_s) {
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0 || tile_s <= 0) return 0;
  // a product that does not fit is reported as no size at all fits
  if (!loom_prod_le({cdiv64(S, tile_s), B, H, D + 1, 4}, (int64_t)1 << 60)) return SIZE_MAX;
  const size_t ns = (size_t)cdiv64(S, tile_s);
  return align256(ns * B * H * sizeof(float)) + ns * B * H * D * sizeof(float);
}

int loom_hip_flash_decode(const void* k, const void* v, const void* q, void* out,
                          void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                          int64_t D, int64_t S, float scale, int64_t tile_b, int64_t tile_s,
                          int64_t tile_n, void* stream, char* err, size_t errlen) {
  return flash_decode_impl<false>(k, v, q, out, workspace, workspace_bytes, B, H, D, S, scale,
                                  tile_b, tile_s, tile_n, stream, err, errlen);
}
int loom_hip_flash_decode_f16(const void* k, const void* v, const void* q, void* out,
                              void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                              int64_t D, int64_t S, float scale, int64_t tile_b, int64_t tile_s,
                              int64_t tile_n, void* stream, char* err, size_t errlen) {
  return flash_decode_impl<true>(k, v, q, out, workspace, workspace_bytes, B, H, D, S, scale,
                                 tile_b, tile_s, tile_n, stream, err, errlen);
}

}  // extern "C"
