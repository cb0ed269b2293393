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
// in: each wave walks 64-key blocks, pulling K and V straight into
// registers with raw buffer loads, and builds the MFMA operands with
// register transposes (v_perm_b32):
//   S^T[key, head] = K^T . Q^T  -- A operand from 8-byte K loads (four keys
//                                 of eight d rows) transposed 8x4
//   O^T[d, head]  += V^T . P^T  -- B operand P^T comes straight from the
//                                 S^T accumulators, A operand V^T from
//                                 16-byte V row loads transposed.
// Keys are permuted inside a block and the permutation is undone only where
// results are addressed, which is sound because softmax and P.V do not
// depend on the order of the keys.  Softmax runs in the log2 domain in fp32.
// One workgroup (4 waves) per (batch, split); the waves' partial states
// are merged through LDS into (lse_s, o_s), exactly the reference's
// gathered tensors; a second kernel performs the split-0 combine.
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
  float c2;    // scale * log2(e)
};

// Split-0 combine of the reference (:147-199), one wave per (b, head):
// lane s < 64 holds lse_s, M = max_s lse_s and den = sum_s exp(lse_s - M)
// are wave reductions, then every lane accumulates out[d] = sum_s w_s o_s[d]
// (w_s = exp(lse_s - M) / den, ascending s) for its D/64 values of d with
// eight splits' loads in flight at a time.  Splits beyond 64 are taken in
// chunks of 64.
template <int D, bool F16>
__global__ void __launch_bounds__(256) decode_combine_kernel(DecodeParams p) {
  constexpr int DPL = D / 64;  // d values per lane
  const int lane = threadIdx.x & 63;
  const int64_t BH = (int64_t)p.B * p.H;
  const int64_t bh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= BH) return;
  const int ns = p.ns;
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, p.lse[s * BH + bh]);
  M = wave_max(M);
  float den = 0.f;
  for (int s = lane; s < ns; s += 64) den += expf(p.lse[s * BH + bh] - M);
  den = wave_sum(den);
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  for (int c0 = 0; c0 < ns; c0 += 64) {
    const int sl = c0 + lane;
    const float wl = sl < ns ? expf(p.lse[sl * BH + bh] - M) / den : 0.f;
    const int cn = min(64, ns - c0);
    for (int u0 = 0; u0 < cn; u0 += 8) {
      float v[8][DPL];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = c0 + min(u0 + u, cn - 1);  // clamped: weight 0 past the end
        const float* src = p.o + (s * BH + bh) * D + lane * DPL;
#pragma unroll
        for (int i = 0; i < DPL; ++i) v[u][i] = src[i];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float w = u0 + u < cn ? __shfl(wl, u0 + u) : 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] += v[u][i] * w;
      }
    }
  }
  uint16_t* dst = p.out + bh * D + lane * DPL;
  if constexpr (DPL == 2)
    *reinterpret_cast<uint32_t*>(dst) = pack2<F16>(acc[0], acc[1]);
  else
    dst[0] = (uint16_t)cvt16<F16>(acc[0]);
}

// D = head dim (64 or 128), HT = head tiles of 16, ALIGNED = S is a
// multiple of 4 (8-byte K chunks start on 8-byte boundaries).
//
// Each wave walks its 64-key blocks as NSTEPS load steps of eight loads:
// DSTEPS steps of K (eight d rows x 4 keys per lane, 8-byte loads) then two
// steps of V (eight keys x VEC d per lane).  Loads run one step ahead of the
// math through a two-slot register ring, continuing into the wave's next
// block; with two waves per SIMD the other wave's math covers the rest of
// the latency.  All loads are raw buffer loads: anything past the tensor
// reads as zero, and keys past the split end are masked to -inf before the
// softmax (so their V rows are multiplied by exactly 0).
template <int D, int HT, bool ALIGNED, bool F16>
__global__ void __launch_bounds__(64 * kWaves) decode_split_kernel(DecodeParams p) {
  constexpr int VEC = D / 16;     // d values per lane per V row, also # of d tiles
  constexpr int DSTEPS = D / 32;  // 32-deep MFMA steps over d
  constexpr int NSTEPS = DSTEPS + 2;
#ifndef LOOM_DECODE_RING
#define LOOM_DECODE_RING 3
#endif
  // ring slots (a divisor of the step count)
  constexpr int R = NSTEPS % LOOM_DECODE_RING == 0 ? LOOM_DECODE_RING : 2;
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
  const int s0 = split * p.tile_s;
  const int s1 = min(S, s0 + p.tile_s);
  const int nblk = (s1 - s0 + kBlockKeys - 1) / kBlockKeys;

  const rsrc_t krs = make_rsrc(p.k + (int64_t)b * D * S, (uint32_t)(D * S * 2));
  const rsrc_t vrs = make_rsrc(p.v + (int64_t)b * S * D, (uint32_t)(S * D * 2));
  const uint16_t* __restrict__ qb = p.q + (int64_t)b * H * D;

  // Q^T operands, shared by the waves through LDS: slot [ds][ht][lane]
  // holds q[h = r + 16 ht][32 ds + 8 g .. +7]
  __shared__ u32x4_t sm_q[DSTEPS][HT][64];
  for (int e = threadIdx.x; e < DSTEPS * HT * 64; e += 64 * kWaves) {
    const int ln = e & 63, ht = (e >> 6) % HT, ds = (e >> 6) / HT;
    const int h = (ln & 15) + 16 * ht;
    sm_q[ds][ht][ln] = h < H ? *reinterpret_cast<const u32x4_t*>(qb + (int64_t)h * D + ds * 32 +
                                                                  (ln >> 4) * 8)
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
        if constexpr (ALIGNED) {
          const u32x2_t w = buf_load8(krs, o);
          buf[e] = u32x4_t{w[0], w[1], 0u, 0u};
        } else {
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
        const uint32_t o = valid ? ((uint32_t)key * D + r * VEC) * 2 : kNone;
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

template <int D, int HT, bool F16>
void launch_split(const DecodeParams& p, bool aligned, hipStream_t st) {
  const dim3 grid(p.ns, p.B), block(64 * kWaves);
  if (aligned)
    hipLaunchKernelGGL((decode_split_kernel<D, HT, true, F16>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((decode_split_kernel<D, HT, false, F16>), grid, block, 0, st, p);
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
  if (!(D == 64 || D == 128))
    return loom_fail(err, errlen, LOOM_EUNSUP, "flash_decode: head_dim %lld not built (64, 128)",
                     (long long)D);
  if (H > 32)
    return loom_fail(err, errlen, LOOM_EUNSUP, "flash_decode: at most 32 query heads (got %lld)",
                     (long long)H);
  if (S * D * 2 > 0x7fffffffll || B > 65535)
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
  p.c2 = scale * 1.4426950408889634f;
  const bool al = S % 4 == 0;
  if (loom_validate_only()) return loom_ok(err, errlen);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 128) {
    if (H > 16) launch_split<128, 2, F16>(p, al, st); else launch_split<128, 1, F16>(p, al, st);
  } else {
    if (H > 16) launch_split<64, 2, F16>(p, al, st); else launch_split<64, 1, F16>(p, al, st);
  }
  int rc = loom_check_launch(err, errlen, "flash_decode (split)");
  if (rc) return rc;
  const dim3 cgrid((unsigned)cdiv64(B * H, 4)), cblock(256);
  if (D == 128)
    hipLaunchKernelGGL((decode_combine_kernel<128, F16>), cgrid, cblock, 0, st, p);
  else
    hipLaunchKernelGGL((decode_combine_kernel<64, F16>), cgrid, cblock, 0, st, p);
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
  std::call_once(g_scratch_once[dev], [dev] {
    int cur = 0;
    hipError_t r = hipGetDevice(&cur);
    if (r == hipSuccess && cur != dev) r = hipSetDevice(dev);
    void* ptr = nullptr;
    if (r == hipSuccess) r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    g_scratch[dev] = ptr;
    g_scratch_rc[dev] = r;
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
