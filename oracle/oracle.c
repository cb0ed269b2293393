/*
 * oracle.c -- fp32 CPU restatement of the six loom-dataflow example kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels in
 * loom-dataflow_amd/csrc: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path never calls it.
 *
 * Each function restates the tensor-level MLIR the Helion frontend emitted
 * for one example (stage 00 of /root/reference/examples/<k>/IR), following
 * the tile structure wherever the tile structure changes the numbers:
 *   - split-K keeps its K-slab partials G[s] (the loom.gather target) and
 *     sums them in ascending s;
 *   - flash_decode keeps its split-KV partials (lse_s, o_s) and the combine;
 *   - attention / flash_decode run the online softmax tile by tile, with the
 *     reference's initial state (m = -inf, l = 1, acc = 0);
 *   - the mamba k-loop adds one fresh partial product per tile_k step.
 * Deliberate differences from the reference (which computes in f16):
 *   - 16-bit storage in bf16 by default, or in IEEE f16 -- the reference's
 *     own element type -- after loom_oracle_set_element_type(1); fp32
 *     arithmetic everywhere (the reference accumulates in f16), one
 *     round-to-nearest-even per 16-bit output element;
 *   - attention gains a `causal` flag (key j visible to query i iff j <= i);
 *   - mamba applies the Mamba-2 intra-chunk causal mask (k <= m) with a select,
 *     and generalises the reference's hard-coded group index h/8 to
 *     h / (H/G).
 * Tiles that overhang a tensor are clamped to the tensor (the reference's
 * subviews would read out of bounds there).
 *
 * Parity of every exported function is pinned in tests/test_oracle.py against
 * fp64 numpy brute force, closed forms and (for mamba) the sequential SSM
 * recurrence; see the header of that file for the list.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))
#define HOT __attribute__((target_clones("avx512f", "avx2", "default")))

/* ------------------------------------------------------------------------ */
/* 16-bit element helpers.  The restated functions read and write their     */
/* 16-bit tensors through elt2f / f2elt, whose format is bf16 (default) or    */
/* IEEE binary16 (the reference's own f16), set by                           */
/* loom_oracle_set_element_type.  Both round to nearest even.                 */
/* ------------------------------------------------------------------------ */

static inline float bf16_bits_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* binary16 -> fp32, exact (IEEE 754-2008 3.6: 1 sign, 5 exponent bits with
   bias 15, 10 fraction bits; exponent 0 = subnormal, 31 = inf/NaN) */
static inline float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    const float v = ldexpf((float)m, -24); /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) u = sign | 0x7f800000u | (m << 13);
  else u = sign | ((e + 112u) << 23) | (m << 13); /* rebias 15 -> 127 */
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> binary16, round to nearest even; overflow to +-inf, NaN quieted */
static inline uint16_t f32_to_f16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  /* 65520 = 65504 + half an ulp and above rounds to infinity */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a >= 0x38800000u) { /* normal: |f| >= 2^-14 */
    const uint32_t r = a + 0xfffu + ((a >> 13) & 1u); /* round the 13 dropped bits */
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13)); /* rebias 127 -> 15 */
  }
  /* subnormal (or zero): an integer multiple of 2^-24; |f| * 2^24 < 1024
     is exact, rintf rounds it to nearest even */
  float af;
  memcpy(&af, &a, 4);
  return (uint16_t)(sign | (uint16_t)rintf(af * 16777216.0f));
}

static int g_elem_f16 = 0;

EXPORT void loom_oracle_set_element_type(int f16) { g_elem_f16 = f16 != 0; }
EXPORT int loom_oracle_element_type(void) { return g_elem_f16; }

static inline float elt2f(uint16_t h) {
  return g_elem_f16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}
static inline uint16_t f2elt(float f) {
  return g_elem_f16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
}

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }

EXPORT void loom_oracle_widen16(const uint16_t *in, float *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = elt2f(in[i]);
}

EXPORT void loom_oracle_round16(const float *in, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = f2elt(in[i]);
}

EXPORT int loom_oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* GEMM core: C[M,N] (fp32) = sum_k A[M,K] * B[K,N], k ascending per element. */
/* A and B already widened to fp32, row-major with leading dims lda/ldb.      */
/* ------------------------------------------------------------------------ */

#define GB_M 32
#define GB_N 256

HOT static void gemm_block_f32(const float *A, int64_t lda, const float *B, int64_t ldb,
                               float *acc, int64_t mb, int64_t nb, int64_t k0, int64_t k1) {
  /* acc is mb x nb, row stride GB_N, accumulated in place */
  for (int64_t i = 0; i < mb; ++i) {
    float *arow = acc + i * GB_N;
    const float *ai = A + i * lda;
    for (int64_t k = k0; k < k1; ++k) {
      const float a = ai[k];
      const float *bk = B + k * ldb;
      for (int64_t j = 0; j < nb; ++j) arow[j] += a * bk[j];
    }
  }
}

/* out_f32 (or out_bf16) = A.B over the K range [k0, k1) for the M x N problem */
static void gemm_range(const float *A, int64_t lda, const float *B, int64_t ldb,
                       int64_t M, int64_t N, int64_t k0, int64_t k1,
                       float *out_f32, uint16_t *out_bf16, int64_t ldo) {
  const int64_t nbm = cdiv(M, GB_M), nbn = cdiv(N, GB_N);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t bi = 0; bi < nbm; ++bi) {
    for (int64_t bj = 0; bj < nbn; ++bj) {
      float acc[GB_M * GB_N];
      const int64_t i0 = bi * GB_M, j0 = bj * GB_N;
      const int64_t mb = min64(GB_M, M - i0), nb = min64(GB_N, N - j0);
      for (int64_t i = 0; i < mb; ++i)
        for (int64_t j = 0; j < nb; ++j) acc[i * GB_N + j] = 0.0f;
      gemm_block_f32(A + i0 * lda, lda, B + j0, ldb, acc, mb, nb, k0, k1);
      for (int64_t i = 0; i < mb; ++i)
        for (int64_t j = 0; j < nb; ++j) {
          const float v = acc[i * GB_N + j];
          if (out_f32) out_f32[(i0 + i) * ldo + j0 + j] = v;
          if (out_bf16) out_bf16[(i0 + i) * ldo + j0 + j] = f2elt(v);
        }
    }
  }
}

static int tiles_ok(int64_t t, int64_t extent) { return t > 0 && t <= extent; }

/*
 * @matmul -- examples/mm/IR/00_from_helion_frontend.mlir:2-35.
 * Grid ceil(M/tile_m) x ceil(N/tile_n) (:11-13); the K loop (:16-27) runs
 * linalg.matmul into a zero-filled accumulator (:15,:25), i.e. every output
 * element is sum_k x[i,k]*y[k,j] in ascending k; one copy-out (:30-32).
 * Because that order does not depend on the tile sizes, tiles are only
 * validated here.
 */
EXPORT int loom_oracle_matmul(const uint16_t *x, const uint16_t *y, uint16_t *out,
                              int64_t M, int64_t N, int64_t K,
                              int64_t tile_m, int64_t tile_n, int64_t tile_k) {
  if (!tiles_ok(tile_m, M) || !tiles_ok(tile_n, N) || !tiles_ok(tile_k, K)) return 1;
  float *A = (float *)malloc(sizeof(float) * M * K);
  float *B = (float *)malloc(sizeof(float) * K * N);
  if (!A || !B) { free(A); free(B); return 2; }
  loom_oracle_widen16(x, A, M * K);
  loom_oracle_widen16(y, B, K * N);
  gemm_range(A, K, B, N, M, N, 0, K, NULL, out, N);
  free(A);
  free(B);
  return 0;
}

/*
 * @batch_matmul -- examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4-44.
 * Grid over (b, m, n) tiles (:10); the K loop (:13-35) accumulates each
 * tile's batch_matmul into the running sum (canonicalized to a direct
 * accumulation in examples/bmm_2Dmesh/IR/01_tensor_canonicalized.mlir:20).
 */
EXPORT int loom_oracle_batch_matmul(const uint16_t *a0, const uint16_t *a1, uint16_t *a2,
                                    int64_t Bt, int64_t M, int64_t N, int64_t K,
                                    int64_t tile_b, int64_t tile_m, int64_t tile_n,
                                    int64_t tile_k) {
  if (!tiles_ok(tile_b, Bt) || !tiles_ok(tile_m, M) || !tiles_ok(tile_n, N) ||
      !tiles_ok(tile_k, K))
    return 1;
  float *A = (float *)malloc(sizeof(float) * M * K);
  float *B = (float *)malloc(sizeof(float) * K * N);
  if (!A || !B) { free(A); free(B); return 2; }
  for (int64_t b = 0; b < Bt; ++b) {
    loom_oracle_widen16(a0 + b * M * K, A, M * K);
    loom_oracle_widen16(a1 + b * K * N, B, K * N);
    gemm_range(A, K, B, N, M, N, 0, K, NULL, a2 + b * M * N, N);
  }
  free(A);
  free(B);
  return 0;
}

/*
 * @split_k_matmul_gather -- examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2-56.
 * Grid (m, n, s) (:12); program s computes the partial P_s of its K slab
 * [s*tile_k, (s+1)*tile_k) into a fresh zero tile (:26-28) and loom.gather
 * stacks it at index s of the gathered buffer (:30-33).  The program with
 * s == 0 reduces the gathered stack over s in index order (:34-46) and stores
 * (:47-51).  Here the gathered buffer for every (m, n) tile is the slice of
 * one [S, M, N] fp32 array `partials` (S = ceil(K/tile_k)).
 */
EXPORT int loom_oracle_split_k_matmul_gather(const uint16_t *a, const uint16_t *b,
                                             uint16_t *out, float *partials,
                                             int64_t M, int64_t N, int64_t K,
                                             int64_t tile_m, int64_t tile_n,
                                             int64_t tile_k) {
  if (!tiles_ok(tile_m, M) || !tiles_ok(tile_n, N) || !tiles_ok(tile_k, K)) return 1;
  const int64_t S = cdiv(K, tile_k);
  float *A = (float *)malloc(sizeof(float) * M * K);
  float *B = (float *)malloc(sizeof(float) * K * N);
  if (!A || !B) { free(A); free(B); return 2; }
  loom_oracle_widen16(a, A, M * K);
  loom_oracle_widen16(b, B, K * N);
  for (int64_t s = 0; s < S; ++s) {
    const int64_t k0 = s * tile_k, k1 = min64(K, k0 + tile_k);
    gemm_range(A, K, B, N, M, N, k0, k1, partials + s * M * N, NULL, N);
  }
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < M * N; ++e) {
    float acc = 0.0f;
    for (int64_t s = 0; s < S; ++s) acc += partials[s * M * N + e];
    out[e] = f2elt(acc);
  }
  free(A);
  free(B);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Online softmax over one tile of keys, shared by attention and decode.     */
/* ------------------------------------------------------------------------ */

/*
 * One step of the reference's KV loop body for `rows` query rows
 * (examples/flashattn/IR/00_from_helion_frontend.mlir:36-113, identical in
 * examples/mqa_decode/IR/00_from_helion_frontend.mlir:42-120):
 *   S = q.k                        (:38)
 *   m_ij = rowmax(S) * scale       (:39-48)
 *   m' = m > m_ij ? m : m_ij       (:49-54, cmpf ogt + select)
 *   P = exp(S*scale - m')          (:55-70)
 *   alpha = exp(m - m')            (:77-86)
 *   l' = l*alpha + rowsum(P)       (:87-96)
 *   acc' = acc*alpha + P.V         (:97-113)
 * S is scores[rows][nk] (raw q.k, masked entries = -inf); V rows are v[nk][D].
 */
static void online_softmax_step(const float *scores, int64_t rows, int64_t nk, int64_t lds,
                                const float *v, int64_t D, float scale,
                                float *m, float *l, float *acc, float *P) {
  for (int64_t i = 0; i < rows; ++i) {
    const float *si = scores + i * lds;
    float mx = -INFINITY;
    for (int64_t n = 0; n < nk; ++n) mx = fmaxf(mx, si[n]);
    const float mij = mx * scale;
    const float mnew = (m[i] > mij) ? m[i] : mij;
    float rs = 0.0f;
    for (int64_t n = 0; n < nk; ++n) {
      const float p = expf(si[n] * scale - mnew);
      P[n] = p;
      rs += p;
    }
    const float alpha = expf(m[i] - mnew);
    l[i] = l[i] * alpha + rs;
    float *ai = acc + i * D;
    for (int64_t d = 0; d < D; ++d) ai[d] *= alpha;
    for (int64_t n = 0; n < nk; ++n) {
      const float p = P[n];
      const float *vn = v + n * D;
      for (int64_t d = 0; d < D; ++d) ai[d] += p * vn[d];
    }
    m[i] = mnew;
  }
}

/*
 * @attention -- examples/flashattn/IR/00_from_helion_frontend.mlir:4-127.
 * k is [BH, D, Skv] (keys transposed), v is [BH, Skv, D], q and out are
 * [BH, Sq, D].  Grid (bh-tile, m-tile) (:16-18); per program the running
 * state starts at m = -inf, l = 1, acc = 0 (:19-23); the KV loop (:28-115)
 * runs online_softmax_step over tiles of tile_n keys; out = acc / l
 * (:116-121).  `causal` (not in the reference) masks key j > query i to
 * -inf before the row max and skips tiles that are fully masked; it needs
 * Sq == Skv.
 */
EXPORT int loom_oracle_attention(const uint16_t *k, const uint16_t *v, const uint16_t *q,
                                 uint16_t *out, int64_t BH, int64_t Sq, int64_t Skv,
                                 int64_t D, float scale, int causal, int64_t tile_b,
                                 int64_t tile_m, int64_t tile_n) {
  if (!tiles_ok(tile_b, BH) || !tiles_ok(tile_m, Sq) || !tiles_ok(tile_n, Skv)) return 1;
  if (causal && Sq != Skv) return 1;
  const int64_t nmt = cdiv(Sq, tile_m);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t bh = 0; bh < BH; ++bh) {
    for (int64_t mt = 0; mt < nmt; ++mt) {
      const int64_t i0 = mt * tile_m, rows = min64(tile_m, Sq - i0);
      float *Q = (float *)malloc(sizeof(float) * rows * D);
      float *S = (float *)malloc(sizeof(float) * rows * tile_n);
      float *Vt = (float *)malloc(sizeof(float) * tile_n * D);
      float *Kt = (float *)malloc(sizeof(float) * D * tile_n);
      float *acc = (float *)calloc(rows * D, sizeof(float));
      float *m = (float *)malloc(sizeof(float) * rows);
      float *l = (float *)malloc(sizeof(float) * rows);
      float *P = (float *)malloc(sizeof(float) * tile_n);
      const uint16_t *qb = q + (bh * Sq + i0) * D;
      for (int64_t e = 0; e < rows * D; ++e) Q[e] = elt2f(qb[e]);
      for (int64_t i = 0; i < rows; ++i) { m[i] = -INFINITY; l[i] = 1.0f; }
      const int64_t nkt = cdiv(Skv, tile_n);
      for (int64_t kt = 0; kt < nkt; ++kt) {
        const int64_t j0 = kt * tile_n, nk = min64(tile_n, Skv - j0);
        if (causal && j0 > i0 + rows - 1) break; /* every key of the tile is masked */
        for (int64_t d = 0; d < D; ++d) {
          const uint16_t *kr = k + (bh * D + d) * Skv + j0;
          for (int64_t n = 0; n < nk; ++n) Kt[d * tile_n + n] = elt2f(kr[n]);
        }
        for (int64_t n = 0; n < nk; ++n) {
          const uint16_t *vr = v + (bh * Skv + j0 + n) * D;
          for (int64_t d = 0; d < D; ++d) Vt[n * D + d] = elt2f(vr[d]);
        }
        for (int64_t i = 0; i < rows; ++i) {
          float *si = S + i * tile_n;
          for (int64_t n = 0; n < nk; ++n) si[n] = 0.0f;
          for (int64_t d = 0; d < D; ++d) {
            const float a = Q[i * D + d];
            const float *kd = Kt + d * tile_n;
            for (int64_t n = 0; n < nk; ++n) si[n] += a * kd[n];
          }
          if (causal)
            for (int64_t n = 0; n < nk; ++n)
              if (j0 + n > i0 + i) si[n] = -INFINITY;
        }
        online_softmax_step(S, rows, nk, tile_n, Vt, D, scale, m, l, acc, P);
      }
      uint16_t *ob = out + (bh * Sq + i0) * D;
      for (int64_t i = 0; i < rows; ++i)
        for (int64_t d = 0; d < D; ++d) ob[i * D + d] = f2elt(acc[i * D + d] / l[i]);
      free(Q); free(S); free(Vt); free(Kt); free(acc); free(m); free(l); free(P);
    }
  }
  return 0;
}

/*
 * @flash_decode -- examples/mqa_decode/IR/00_from_helion_frontend.mlir:6-202.
 * k is [B, D, S] (transposed), v is [B, S, D], q and out are [B, H, D]: H
 * query heads share one KV head.  Grid (b-tile, split) (:19-21); split s
 * covers keys [s*tile_s, (s+1)*tile_s) in steps of tile_n (:30-36) with the
 * same online softmax; then lse_s = log(l) + m (:123-132), o_s = acc / l
 * (:133-138), both gathered at index s (:139-146) -- here into
 * lse_ws[nsplit, B, H] and o_ws[nsplit, B, H, D].  Split 0 combines
 * (:147-199): M = max_s lse_s, w_s = exp(lse_s - M) / sum_s exp(lse_s - M),
 * out = sum_s w_s * o_s in ascending s.  The i64 argmax computed at
 * :149-159 is never used and is omitted.
 */
EXPORT int loom_oracle_flash_decode(const uint16_t *k, const uint16_t *v, const uint16_t *q,
                                    uint16_t *out, float *lse_ws, float *o_ws,
                                    int64_t B, int64_t H, int64_t D, int64_t S, float scale,
                                    int64_t tile_b, int64_t tile_s, int64_t tile_n) {
  if (!tiles_ok(tile_b, B) || !tiles_ok(tile_s, S) || !tiles_ok(tile_n, S)) return 1;
  if (D > 1024) return 1;
  const int64_t ns = cdiv(S, tile_s);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t s = 0; s < ns; ++s) {
      float *Q = (float *)malloc(sizeof(float) * H * D);
      float *Sc = (float *)malloc(sizeof(float) * H * tile_n);
      float *Kt = (float *)malloc(sizeof(float) * D * tile_n);
      float *Vt = (float *)malloc(sizeof(float) * tile_n * D);
      float *acc = (float *)calloc(H * D, sizeof(float));
      float *m = (float *)malloc(sizeof(float) * H);
      float *l = (float *)malloc(sizeof(float) * H);
      float *P = (float *)malloc(sizeof(float) * tile_n);
      for (int64_t e = 0; e < H * D; ++e) Q[e] = elt2f(q[b * H * D + e]);
      for (int64_t h = 0; h < H; ++h) { m[h] = -INFINITY; l[h] = 1.0f; }
      const int64_t s0 = s * tile_s, s1 = min64(S, s0 + tile_s);
      for (int64_t j0 = s0; j0 < s1; j0 += tile_n) {
        const int64_t nk = min64(tile_n, s1 - j0);
        for (int64_t d = 0; d < D; ++d) {
          const uint16_t *kr = k + (b * D + d) * S + j0;
          for (int64_t n = 0; n < nk; ++n) Kt[d * tile_n + n] = elt2f(kr[n]);
        }
        for (int64_t n = 0; n < nk; ++n) {
          const uint16_t *vr = v + (b * S + j0 + n) * D;
          for (int64_t d = 0; d < D; ++d) Vt[n * D + d] = elt2f(vr[d]);
        }
        for (int64_t h = 0; h < H; ++h) {
          float *sh = Sc + h * tile_n;
          for (int64_t n = 0; n < nk; ++n) sh[n] = 0.0f;
          for (int64_t d = 0; d < D; ++d) {
            const float a = Q[h * D + d];
            const float *kd = Kt + d * tile_n;
            for (int64_t n = 0; n < nk; ++n) sh[n] += a * kd[n];
          }
        }
        online_softmax_step(Sc, H, nk, tile_n, Vt, D, scale, m, l, acc, P);
      }
      for (int64_t h = 0; h < H; ++h) {
        lse_ws[(s * B + b) * H + h] = logf(l[h]) + m[h];
        for (int64_t d = 0; d < D; ++d)
          o_ws[((s * B + b) * H + h) * D + d] = acc[h * D + d] / l[h];
      }
      free(Q); free(Sc); free(Kt); free(Vt); free(acc); free(m); free(l); free(P);
    }
  }
  /* combine (split 0's program), per batch and head */
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      float M = -INFINITY;
      for (int64_t s = 0; s < ns; ++s) M = fmaxf(M, lse_ws[(s * B + b) * H + h]);
      float den = 0.0f;
      for (int64_t s = 0; s < ns; ++s) den += expf(lse_ws[(s * B + b) * H + h] - M);
      float o[1024];
      const int64_t Dc = D < 1024 ? D : 1024;
      for (int64_t d = 0; d < Dc; ++d) o[d] = 0.0f;
      for (int64_t s = 0; s < ns; ++s) {
        const float w = expf(lse_ws[(s * B + b) * H + h] - M) / den;
        const float *os = o_ws + ((s * B + b) * H + h) * D;
        for (int64_t d = 0; d < Dc; ++d) o[d] += os[d] * w;
      }
      for (int64_t d = 0; d < Dc; ++d) out[(b * H + h) * D + d] = f2elt(o[d]);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Mamba-2 SSD                                                               */
/* ------------------------------------------------------------------------ */

/*
 * @helion_mamba2_chunk_scan_kernel --
 * examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4-126
 * (fused form examples/mamba_chunk_scan/IR/01_tensor_canonicalized.mlir:55-106).
 * Shapes: cb [b,c,G,Q,Q] bf16; x [b,H,L,P] bf16; dt, dA_cumsum [b,H,c,Q]
 * fp32; C [b,G,L,N] bf16; D [H] fp32; prev_states_T [b,c,H,N,P] fp32;
 * out [b,H,L,P] bf16, L = c*Q.  For each (b, h, c) and output tile
 * (m-tile, p-tile):
 *   acc = (C[m,:] . prevT[:,p]) * exp(dA[m])                (:46-56)
 *   for each k tile (:57-104):
 *     W[m,k] = cb[m,k] * exp(dA[m] - dA[k]) * dt[k]         (:61-93)
 *     acc += W . x[k,p]   (fresh partial, then added)       (:97-102)
 *   out = acc + x[m,p] * D[h]                               (:105-121)
 * with the k <= m mask (a select, the reference has none) and g = h/(H/G)
 * (the reference hard-codes h/8 at :43).  tile_b/tile_h/tile_c must be 1.
 */
EXPORT int loom_oracle_mamba_chunk_scan(const uint16_t *cb, const uint16_t *x, const float *dt,
                                        const float *dA, const uint16_t *C, const float *Dh,
                                        const float *prevT, uint16_t *out,
                                        int64_t Bb, int64_t nc, int64_t Hh, int64_t G,
                                        int64_t Q, int64_t P, int64_t N,
                                        int64_t tile_m, int64_t tile_n, int64_t tile_k) {
  if (!tiles_ok(tile_m, Q) || !tiles_ok(tile_n, P) || tile_k <= 0) return 1;
  if (G <= 0 || Hh % G != 0) return 1;
  const int64_t L = nc * Q, hpg = Hh / G;
  const int64_t nmt = cdiv(Q, tile_m), npt = cdiv(P, tile_n);
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int64_t b = 0; b < Bb; ++b) {
    for (int64_t h = 0; h < Hh; ++h) {
      for (int64_t c = 0; c < nc; ++c) {
        const int64_t g = h / hpg;
        const float *dAc = dA + ((b * Hh + h) * nc + c) * Q;
        const float *dtc = dt + ((b * Hh + h) * nc + c) * Q;
        const uint16_t *cbc = cb + (((b * nc + c) * G + g) * Q) * Q;
        const uint16_t *xc = x + ((b * Hh + h) * L + c * Q) * P;
        const uint16_t *Cc = C + ((b * G + g) * L + c * Q) * N;
        const float *pv = prevT + (((b * nc + c) * Hh + h) * N) * P;
        uint16_t *oc = out + ((b * Hh + h) * L + c * Q) * P;
        float *acc = (float *)malloc(sizeof(float) * tile_m * tile_n);
        float *part = (float *)malloc(sizeof(float) * tile_m * tile_n);
        float *W = (float *)malloc(sizeof(float) * tile_m * tile_k);
        for (int64_t mt = 0; mt < nmt; ++mt) {
          const int64_t m0 = mt * tile_m, rows = min64(tile_m, Q - m0);
          for (int64_t pt = 0; pt < npt; ++pt) {
            const int64_t p0 = pt * tile_n, cols = min64(tile_n, P - p0);
            for (int64_t i = 0; i < rows; ++i) {
              const float e = expf(dAc[m0 + i]);
              for (int64_t j = 0; j < cols; ++j) {
                float s = 0.0f;
                for (int64_t n = 0; n < N; ++n)
                  s += elt2f(Cc[(m0 + i) * N + n]) * pv[n * P + p0 + j];
                acc[i * tile_n + j] = s * e;
              }
            }
            /* k tiles up to ceil((mt+1)*tile_m / tile_k), clamped to Q */
            const int64_t kend = min64(Q, cdiv((mt + 1) * tile_m, tile_k) * tile_k);
            for (int64_t k0 = 0; k0 < kend; k0 += tile_k) {
              const int64_t nk = min64(tile_k, kend - k0);
              for (int64_t i = 0; i < rows; ++i) {
                const int64_t mi = m0 + i;
                for (int64_t kk = 0; kk < nk; ++kk) {
                  const int64_t ki = k0 + kk;
                  float w = 0.0f;
                  if (ki <= mi) {
                    const float decay = expf(dAc[mi] - dAc[ki]);
                    w = elt2f(cbc[mi * Q + ki]) * decay;
                    w = w * dtc[ki];
                  }
                  W[i * tile_k + kk] = w;
                }
              }
              for (int64_t i = 0; i < rows; ++i)
                for (int64_t j = 0; j < cols; ++j) {
                  float s = 0.0f;
                  for (int64_t kk = 0; kk < nk; ++kk)
                    s += W[i * tile_k + kk] * elt2f(xc[(k0 + kk) * P + p0 + j]);
                  part[i * tile_n + j] = s;
                }
              for (int64_t i = 0; i < rows; ++i)
                for (int64_t j = 0; j < cols; ++j) acc[i * tile_n + j] += part[i * tile_n + j];
            }
            for (int64_t i = 0; i < rows; ++i)
              for (int64_t j = 0; j < cols; ++j) {
                const float xv = elt2f(xc[(m0 + i) * P + p0 + j]);
                oc[(m0 + i) * P + p0 + j] = f2elt(acc[i * tile_n + j] + xv * Dh[h]);
              }
          }
        }
        free(acc);
        free(part);
        free(W);
      }
    }
  }
  return 0;
}

/*
 * SSD prologue: derives chunk_scan's inputs from the raw Mamba-2 inputs
 * (x [b,H,L,P] bf16, dt [b,H,L] fp32 (already softplus'ed), A [H] fp32,
 * B and C [b,G,L,N] bf16).  The reference takes cb, dA_cumsum and
 * prev_states_T as inputs of @helion_mamba2_chunk_scan_kernel
 * (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4); these are
 * the standard Mamba-2 SSD definitions (Dao & Gu 2024, "Transformers are
 * SSMs", Sec. 6), checked in tests/test_oracle.py against the sequential
 * recurrence h_t = exp(dt_t A) h_{t-1} + dt_t B_t x_t^T, y_t = C_t h_t + D x_t.
 *   dt_out[b,h,c,q]       = dt[b,h,cQ+q]
 *   dA_cumsum[b,h,c,q]    = sum_{j<=q} dt[b,h,cQ+j] * A[h]
 *   cb[b,c,g,m,k]         = (k <= m) ? bf16(sum_n C[b,g,cQ+m,n] B[b,g,cQ+k,n]) : 0
 *   states[b,c,h,n,p]     = sum_k B[cQ+k,n] exp(dA_cs[Q-1]-dA_cs[k]) dt[k] x[cQ+k,p]
 *   prevT[b,0]            = 0
 *   prevT[b,c+1]          = exp(dA_cs[c][Q-1]) prevT[b,c] + states[b,c]
 */
EXPORT int loom_oracle_mamba_prologue(const uint16_t *x, const float *dt, const float *A,
                                      const uint16_t *Bm, const uint16_t *C,
                                      float *dt_out, float *dA_cumsum, uint16_t *cb,
                                      float *prevT, int64_t Bb, int64_t nc, int64_t Hh,
                                      int64_t G, int64_t Q, int64_t P, int64_t N) {
  if (G <= 0 || Hh % G != 0) return 1;
  const int64_t L = nc * Q, hpg = Hh / G;
  /* dt re-layout and per-chunk cumulative sum */
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < Bb; ++b)
    for (int64_t h = 0; h < Hh; ++h)
      for (int64_t c = 0; c < nc; ++c) {
        float s = 0.0f;
        for (int64_t qq = 0; qq < Q; ++qq) {
          const float d = dt[(b * Hh + h) * L + c * Q + qq];
          dt_out[((b * Hh + h) * nc + c) * Q + qq] = d;
          s += d * A[h];
          dA_cumsum[((b * Hh + h) * nc + c) * Q + qq] = s;
        }
      }
  /* cb = C B^T per chunk, lower triangular */
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < Bb; ++b)
    for (int64_t c = 0; c < nc; ++c)
      for (int64_t g = 0; g < G; ++g)
        for (int64_t i = 0; i < Q; ++i)
          for (int64_t j = 0; j < Q; ++j) {
            float s = 0.0f;
            if (j <= i)
              for (int64_t n = 0; n < N; ++n)
                s += elt2f(C[((b * G + g) * L + c * Q + i) * N + n]) *
                     elt2f(Bm[((b * G + g) * L + c * Q + j) * N + n]);
            cb[(((b * nc + c) * G + g) * Q + i) * Q + j] = f2elt(s);
          }
  /* chunk states and the sequential inter-chunk pass */
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t b = 0; b < Bb; ++b)
    for (int64_t h = 0; h < Hh; ++h) {
      const int64_t g = h / hpg;
      float *st = (float *)calloc(N * P, sizeof(float));
      float *w = (float *)malloc(sizeof(float) * Q);
      for (int64_t c = 0; c < nc; ++c) {
        float *pv = prevT + (((b * nc + c) * Hh + h) * N) * P;
        if (c == 0) {
          for (int64_t e = 0; e < N * P; ++e) pv[e] = 0.0f;
        } else {
          const float *pp = prevT + (((b * nc + c - 1) * Hh + h) * N) * P;
          const float *dAp = dA_cumsum + ((b * Hh + h) * nc + c - 1) * Q;
          const float decay = expf(dAp[Q - 1]);
          for (int64_t e = 0; e < N * P; ++e) pv[e] = decay * pp[e] + st[e];
        }
        /* states of chunk c (consumed when building chunk c+1) */
        const float *dAc = dA_cumsum + ((b * Hh + h) * nc + c) * Q;
        const float *dtc = dt_out + ((b * Hh + h) * nc + c) * Q;
        for (int64_t kk = 0; kk < Q; ++kk) w[kk] = expf(dAc[Q - 1] - dAc[kk]) * dtc[kk];
        for (int64_t e = 0; e < N * P; ++e) st[e] = 0.0f;
        for (int64_t kk = 0; kk < Q; ++kk) {
          const uint16_t *Br = Bm + ((b * G + g) * L + c * Q + kk) * N;
          const uint16_t *xr = x + ((b * Hh + h) * L + c * Q + kk) * P;
          for (int64_t n = 0; n < N; ++n) {
            const float bw = elt2f(Br[n]) * w[kk];
            for (int64_t p = 0; p < P; ++p) st[n * P + p] += bw * elt2f(xr[p]);
          }
        }
      }
      free(st);
      free(w);
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs: the counter-based generator of the measurement          */
/* protocol (splitmix64 -> uniform, Box-Muller -> normal, round-to-nearest-  */
/* even -> bf16), so the CPU baseline and the GPU harness can make the same  */
/* tensors without sharing memory or a framework's random stream.  Not part */
/* of the reference.  loom-dataflow_amd/csrc/synth.hip computes the same     */
/* values on the GPU with the same operations in the same order (every       */
/* multiply-add an explicit fmaf, division correctly rounded, the square    */
/* root in integer arithmetic), so the two are bit-identical                 */
/* (tests/test_gpu_synth.py).                                               */
/*                                                                          */
/* Element i of stream `seed`: z = mix64(seed * K1 + i * K2) with the        */
/* splitmix64 finaliser; u = top 24 bits of z * 2^-24 (exact).  Normal:      */
/* u1 = (top 24 bits + 1) * 2^-24 in (0, 1], u2 = next 24 bits * 2^-24,      */
/* n = sqrt(-2 ln u1) cos(2 pi u2).  ln: exponent * ln 2 plus the odd        */
/* series of ln((1+s)/(1-s)) on a mantissa in [sqrt(1/2), sqrt(2)); cos(2 pi  */
/* u2): u2 splits exactly into an octant and a fraction of pi/4, then        */
/* Taylor polynomials of sin and cos on [0, pi/4] (errors below 1e-7).       */
/* ------------------------------------------------------------------------ */
static inline uint64_t synth_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline uint64_t synth_bits(uint64_t seed, int64_t i) {
  return synth_mix(seed * 0xD1B54A32D192ED03ull + (uint64_t)i * 0x9E3779B97F4A7C15ull);
}

/* ln x for x in [2^-24, 1] */
static inline float synth_ln(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  int e = (int)((b >> 23) & 0xff) - 127;
  b = (b & 0x007fffffu) | 0x3f800000u;   /* mantissa m in [1, 2) */
  float m;
  memcpy(&m, &b, 4);
  if (m > 1.41421356f) {                 /* m in [sqrt(1/2), sqrt(2)) */
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = fmaf(s2, 0.11111111f, 0.14285715f);   /* 1/9, 1/7 */
  p = fmaf(s2, p, 0.2f);
  p = fmaf(s2, p, 0.33333334f);
  p = fmaf(s2, p, 1.0f);
  const float lnm = 2.0f * s * p;
  return fmaf((float)e, 0.69314718f, lnm);
}

/* sin and cos of a in [0, pi/4] */
static inline float synth_sin(float a) {
  const float a2 = a * a;
  float p = fmaf(a2, -2.5052108e-8f, 2.7557319e-6f);
  p = fmaf(a2, p, -1.9841270e-4f);
  p = fmaf(a2, p, 8.3333333e-3f);
  p = fmaf(a2, p, -1.6666667e-1f);
  return fmaf(a * a2, p, a);
}
static inline float synth_cos(float a) {
  const float a2 = a * a;
  float p = fmaf(a2, 2.0876757e-9f, -2.7557319e-7f);
  p = fmaf(a2, p, 2.4801587e-5f);
  p = fmaf(a2, p, -1.3888889e-3f);
  p = fmaf(a2, p, 4.1666667e-2f);
  p = fmaf(a2, p, -0.5f);
  return fmaf(a2, p, 1.0f);
}

/* cos(2 pi t) for t = k * 2^-24, k in [0, 2^24) */
static inline float synth_cos2pi(float t) {
  const float t8 = t * 8.0f;             /* exact */
  const int o = (int)t8;                 /* octant 0..7 */
  const float f = t8 - (float)o;         /* exact, in [0, 1) */
  const int k = o >> 1;
  if ((o & 1) == 0) {                    /* angle k pi/2 + f pi/4 */
    const float a = f * 0.78539816f;
    switch (k) {
      case 0: return synth_cos(a);
      case 1: return -synth_sin(a);
      case 2: return -synth_cos(a);
      default: return synth_sin(a);
    }
  }
  /* angle (k + 1) pi/2 - (1 - f) pi/4 */
  const float a = (1.0f - f) * 0.78539816f;
  switch (k) {
    case 0: return synth_sin(a);
    case 1: return -synth_cos(a);
    case 2: return -synth_sin(a);
    default: return synth_cos(a);
  }
}

/* sqrt(x) rounded to nearest, for x = 0 or a positive normal float, in integer
   arithmetic (the device's square root instruction is not correctly rounded):
   x = M 2^E with M in [2^24, 2^26) and E even, R = floor(sqrt(M 2^24)) has 25
   bits (a floating-point estimate corrected by integer steps, so any estimate
   works), and the 24-bit significand is R / 2 rounded by R's last bit (a square
   root of a float is never halfway between two floats). */
static inline float synth_sqrt(float x) {
  if (!(x > 0.0f)) return 0.0f;
  uint32_t bx;
  memcpy(&bx, &x, 4);
  uint64_t m = (bx & 0x007fffffu) | 0x00800000u;  /* x = m 2^e, m in [2^23, 2^24) */
  int e = (int)((bx >> 23) & 0xff) - 150;
  if (e & 1) {
    m <<= 1;
    e -= 1;
  } else {
    m <<= 2;
    e -= 2;
  }
  const uint64_t n = m << 24;                      /* [2^48, 2^50) */
  uint64_t r = (uint64_t)sqrt((double)n);
  while (r * r > n) --r;
  while ((r + 1) * (r + 1) <= n) ++r;
  const uint64_t q = (r >> 1) + (r & 1);           /* <= 2^24 */
  return ldexpf((float)q, (e - 24) / 2 + 1);
}

/* value of element i: dist 0 uniform in [a, b), dist 1 normal(a, b) */
static inline float synth_value(uint64_t seed, int64_t i, int dist, float a, float b) {
  const uint64_t z = synth_bits(seed, i);
  if (dist == 0) return fmaf(b - a, (float)(z >> 40) * 0x1p-24f, a);
  const float u1 = (float)((z >> 40) + 1) * 0x1p-24f;
  const float u2 = (float)((z >> 16) & 0xffffffu) * 0x1p-24f;
  const float r = synth_sqrt(-2.0f * synth_ln(u1));
  return fmaf(b, r * synth_cos2pi(u2), a);
}

/* n values into bf16 bits (bf16 = 1) or fp32 (bf16 = 0); dist as above */
EXPORT int loom_oracle_synth(void *out, int64_t n, uint64_t seed, int dist, float a, float b,
                             int bf16) {
  if (!out || n < 0 || (dist != 0 && dist != 1)) return 1;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float v = synth_value(seed, i, dist, a, b);
    if (bf16) ((uint16_t *)out)[i] = f32_to_bf16_bits(v);
    else ((float *)out)[i] = v;
  }
  return 0;
}

/* the generator's square root on n inputs (checked against IEEE sqrtf) */
EXPORT void loom_oracle_synth_sqrt(const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = synth_sqrt(in[i]);
}
