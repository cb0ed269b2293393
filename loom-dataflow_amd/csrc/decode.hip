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
// gfx950 mapping.  Decode is bound by streaming K and V from HBM (the 32
// heads give 32 FLOP per KV byte), so nothing goes through LDS on the way
// in: each wave pulls a 128-key block of K and V straight into registers
// with 16-byte loads (16 lanes cover one 256-byte row, fully coalesced) and
// turns 8x8 blocks into MFMA operands with a register transpose:
//   S^T[key, head] = K^T . Q^T  -- A operand: lane (r, g) holds keys
//                                 base + 8r + j, d-group g (j = tile index)
//   O^T[d, head]  += V^T . P^T  -- B operand P^T comes straight from the
//                                 S^T accumulators of two key tiles, A
//                                 operand V^T from eight V rows transposed.
// Keys and d are permuted inside a block (key = base + 8r + j,
// d = VEC*r + u) and the permutation is undone only where results are
// addressed, which is sound because softmax and P.V do not depend on the
// order of the keys.  Softmax runs in the log2 domain in fp32.
// One workgroup (4 waves) per (batch, split); the waves' partial states
// are merged through LDS into (lse_s, o_s), exactly the reference's
// gathered tensors; a second kernel performs the split-0 combine.
#include "common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kBlockKeys = 128;   // keys per wave step: 16 lanes x 8 keys

struct DecodeParams {
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* q;
  float* lse;  // [ns, B, H]
  float* o;    // [ns, B, H, D]
  int B, H, S, tile_s, ns;
  float c2;    // scale * log2(e)
};

template <int VEC>
struct VRow;
template <>
struct VRow<8> { typedef u32x4_t T; };
template <>
struct VRow<4> { typedef u32x2_t T; };

// D = head dim (64 or 128), HT = head tiles of 16, ALIGNED = S and tile_s
// are multiples of 8 (16-byte K chunks never straddle the split end).
template <int D, int HT, bool ALIGNED>
__global__ void __launch_bounds__(64 * kWaves) decode_split_kernel(DecodeParams p) {
  constexpr int VEC = D / 16;     // d values per lane per V row, also # of d tiles
  constexpr int DSTEPS = D / 32;  // 32-deep MFMA steps over d
  typedef typename VRow<VEC>::T vrow_t;
  constexpr int HP = HT * 16;     // padded head count
  constexpr int ACC_STRIDE = D + 1;
  __shared__ float sm_m[kWaves][HP];
  __shared__ float sm_l[kWaves][HP];
  __shared__ float sm_acc[kWaves][HP * ACC_STRIDE];

  const int split = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int H = p.H, S = p.S;
  const int s0 = split * p.tile_s;
  const int s1 = min(S, s0 + p.tile_s);

  const uint16_t* __restrict__ kb = p.k + (int64_t)b * D * S;
  const uint16_t* __restrict__ vb = p.v + (int64_t)b * S * D;
  const uint16_t* __restrict__ qb = p.q + (int64_t)b * H * D;

  // Q^T operand: lane holds q[h = r + 16 ht][32 ds + 8 g .. +7]
  u32x4_t qf[DSTEPS][HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    const int h = r + 16 * ht;
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds)
      qf[ds][ht] = h < H ? *reinterpret_cast<const u32x4_t*>(qb + (int64_t)h * D + ds * 32 + g * 8)
                         : u32x4_t{0u, 0u, 0u, 0u};
  }

  float m_run[HT], l_run[HT];
  f32x4_t ot[VEC][HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    m_run[ht] = -INFINITY;
    l_run[ht] = 0.f;
#pragma unroll
    for (int u = 0; u < VEC; ++u) ot[u][ht] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int base = s0 + wave * kBlockKeys; base < s1; base += kWaves * kBlockKeys) {
    // ---- S^T = K^T Q^T over the block's 128 keys
    f32x4_t st[8][HT];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) st[j][ht] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int key0 = base + r * 8;  // this lane's 8 keys: key0 .. key0+7
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds) {
      u32x4_t kr[8], kt[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t* row = kb + (int64_t)(ds * 32 + g * 8 + e) * S;
        if constexpr (ALIGNED) {
          kr[e] = key0 < s1 ? *reinterpret_cast<const u32x4_t*>(row + key0)
                            : u32x4_t{0u, 0u, 0u, 0u};
        } else {
          uint32_t h[8];
#pragma unroll
          for (int x = 0; x < 8; ++x) h[x] = key0 + x < s1 ? (uint32_t)row[key0 + x] : 0u;
          kr[e] = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                          h[6] | (h[7] << 16)};
        }
      }
      transpose8x8(kr, kt);  // kt[j] = d values 32ds+8g..+7 of key key0 + j
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) st[j][ht] = mfma16(kt[j], qf[ds][ht], st[j][ht]);
    }

    // ---- online softmax (log2 domain).  st[j][ht][i] is the score of key
    // base + 8*(4g+i) + j for head r + 16 ht.
    float alpha[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = base + 8 * (4 * g + i) + j;
          float t = st[j][ht][i] * p.c2;
          if (key >= s1) t = -INFINITY;
          st[j][ht][i] = t;
          mx = fmaxf(mx, t);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[ht], mx);
      alpha[ht] = fast_exp2(m_run[ht] - m_new);
      m_run[ht] = m_new;
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = fast_exp2(st[j][ht][i] - m_new);
          st[j][ht][i] = pv;
          ls += pv;
        }
      l_run[ht] = l_run[ht] * alpha[ht] + ls;
#pragma unroll
      for (int u = 0; u < VEC; ++u) ot[u][ht] *= alpha[ht];
    }

    // ---- O^T += V^T P^T, 32 keys per MFMA step (tiles j0 = 2c, j1 = 2c+1)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j0 = 2 * c, j1 = 2 * c + 1;
      u32x4_t pf[HT];
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
        pf[ht] = u32x4_t{pack_bf16x2(st[j0][ht][0], st[j0][ht][1]),
                         pack_bf16x2(st[j0][ht][2], st[j0][ht][3]),
                         pack_bf16x2(st[j1][ht][0], st[j1][ht][1]),
                         pack_bf16x2(st[j1][ht][2], st[j1][ht][3])};
      // k slot t of group g: key base + 8*(4g + t%4) + (t<4 ? j0 : j1)
      vrow_t vr[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int key = base + 8 * (4 * g + (t & 3)) + (t < 4 ? j0 : j1);
        if (key < s1)
          vr[t] = *reinterpret_cast<const vrow_t*>(vb + (int64_t)key * D + r * VEC);
        else
          vr[t] = vrow_t{};
      }
      // transpose: va[u] = V[key_t][VEC*r + u] for t = 0..7
      u32x4_t va[VEC];
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t x = vr[2 * i][u / 2], y = vr[2 * i + 1][u / 2];
          va[u][i] = (u & 1) ? pack_hi(x, y) : pack_lo(x, y);
        }
      }
#pragma unroll
      for (int u = 0; u < VEC; ++u)
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) ot[u][ht] = mfma16(va[u], pf[ht], ot[u][ht]);
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
  const int64_t row0 = ((int64_t)split * p.B + b) * H;
  for (int e = threadIdx.x; e < H * D; e += 64 * kWaves) {
    const int h = e / D, d = e % D;
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
    p.o[(row0 + h) * D + d] = o / L;
    if (d == 0) p.lse[row0 + h] = logf(L) + M * 0.69314718055994530942f;
  }
}

// Split-0 combine of the reference (:147-199), one workgroup per (b, head).
__global__ void __launch_bounds__(128) decode_combine_kernel(const float* __restrict__ lse,
                                                             const float* __restrict__ o,
                                                             uint16_t* __restrict__ out,
                                                             int BH, int D, int ns) {
  const int bh = blockIdx.x;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, lse[(int64_t)s * BH + bh]);
  float den = 0.f;
  for (int s = 0; s < ns; ++s) den += expf(lse[(int64_t)s * BH + bh] - M);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (int s = 0; s < ns; ++s) {
      const float w = expf(lse[(int64_t)s * BH + bh] - M) / den;
      acc += o[((int64_t)s * BH + bh) * D + d] * w;
    }
    out[(int64_t)bh * D + d] = (uint16_t)f2bf(acc);
  }
}

template <int D, int HT>
void launch_split(const DecodeParams& p, bool aligned, hipStream_t st) {
  const dim3 grid(p.ns, p.B), block(64 * kWaves);
  if (aligned)
    hipLaunchKernelGGL((decode_split_kernel<D, HT, true>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((decode_split_kernel<D, HT, false>), grid, block, 0, st, p);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

size_t loom_hip_flash_decode_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t S,
                                             int64_t tile_s) {
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0 || tile_s <= 0) return 0;
  const size_t ns = (size_t)cdiv64(S, tile_s);
  return align256(ns * B * H * sizeof(float)) + ns * B * H * D * sizeof(float);
}

int loom_hip_flash_decode(const void* k, const void* v, const void* q, void* out,
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
  if (!(D == 64 || D == 128))
    return loom_fail(err, errlen, LOOM_EUNSUP, "flash_decode: head_dim %lld not built (64, 128)",
                     (long long)D);
  if (H > 32)
    return loom_fail(err, errlen, LOOM_EUNSUP, "flash_decode: at most 32 query heads (got %lld)",
                     (long long)H);
  if (S > (1ll << 30) || B > 65535)
    return loom_fail(err, errlen, LOOM_EINVAL, "flash_decode: S or B too large");
  if (!aligned16(k) || !aligned16(v) || !aligned16(q))
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
  p.o = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                 align256((size_t)ns * B * H * sizeof(float)));
  p.B = (int)B;
  p.H = (int)H;
  p.S = (int)S;
  p.tile_s = (int)tile_s;
  p.ns = (int)ns;
  p.c2 = scale * 1.4426950408889634f;
  const bool al = S % 8 == 0 && tile_s % 8 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 128) {
    if (H > 16) launch_split<128, 2>(p, al, st); else launch_split<128, 1>(p, al, st);
  } else {
    if (H > 16) launch_split<64, 2>(p, al, st); else launch_split<64, 1>(p, al, st);
  }
  int rc = loom_check_launch(err, errlen, "flash_decode (split)");
  if (rc) return rc;
  hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)(B * H)), dim3(128), 0, st, p.lse, p.o,
                     static_cast<uint16_t*>(out), (int)(B * H), (int)D, (int)ns);
  return loom_check_launch(err, errlen, "flash_decode (combine)");
}

}  // extern "C"
